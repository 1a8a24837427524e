"""Pins the CPU oracle (oracle/kvpath_oracle.py) before anything is compared with it.

The reference ships no golden vectors for this path, so each oracle function is checked
against something independent of its own code: brute-force loops over raw storage,
torch's SDPA (with enable_gqa / is_causal), closed forms and invariants.  Each check
names the mistake it is there to catch.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import kvpath_oracle as ref
from tests.helpers import gen, randn_bf16, interleaved_pool, random_block_tables


# ------------------------------------------------------------------------------ append

def _raw_u16(pool: torch.Tensor) -> np.ndarray:
    return pool.view(torch.int16).numpy().view(np.uint16).reshape(-1).copy()


def test_append_writes_interleaved_page_bytes():
    """Byte-level check of the engine page layout: token i with slot s lands in page
    s // bs at element offset (s % bs) * Hkv * D for K and at half a page further for V.
    Catches: wrong block stride (bs*Hkv*D instead of the page), K/V halves swapped,
    slot -> (block, offset) mix-ups, -1 not skipped, neighbouring slots touched."""
    g = gen(1)
    nb, bs, hkv, d, n = 6, 4, 2, 8, 9
    pool, kc, vc = interleaved_pool(nb, bs, hkv, d, g)
    key, value = randn_bf16((n, hkv, d), g), randn_bf16((n, hkv, d), g)
    slots = np.array([5, -1, 0, 23, 7, -1, 12, 4, 19], dtype=np.int32)
    before = _raw_u16(pool)
    ref.kv_append(ref.bf16_bits(key), ref.bf16_bits(value), ref.bf16_bits(kc), ref.bf16_bits(vc), slots)
    after = _raw_u16(pool)

    expect = before.copy()
    page = 2 * bs * hkv * d  # elements per page
    kb, vb = ref.bf16_bits(key), ref.bf16_bits(value)
    for i, s in enumerate(slots):
        if s == -1:
            continue
        for h in range(hkv):
            for e in range(d):
                off = (s // bs) * page + (s % bs) * hkv * d + h * d + e
                expect[off] = kb[i, h, e]
                expect[off + page // 2] = vb[i, h, e]
    assert np.array_equal(after, expect)


def test_append_contiguous_layout_and_row_strides():
    """Contiguous caches and a value tensor that is a strided view of a wider buffer
    (Qwen3's v): the copy follows each tensor's own strides."""
    g = gen(2)
    nb, bs, hkv, d, n = 4, 8, 2, 16, 11
    kc, vc = randn_bf16((nb, bs, hkv, d), g), randn_bf16((nb, bs, hkv, d), g)
    key = randn_bf16((n, hkv, d), g)
    wide = randn_bf16((n, 3 * hkv * d), g)
    value = wide[:, 2 * hkv * d:].view(n, hkv, d)
    slots = torch.randperm(nb * bs, generator=g)[:n].numpy().astype(np.int32)
    slots[[2, 7]] = -1
    k0, v0 = kc.clone(), vc.clone()
    ref.kv_append(ref.bf16_bits(key), ref.bf16_bits(value), ref.bf16_bits(kc), ref.bf16_bits(vc), slots)
    for i, s in enumerate(slots):
        if s == -1:
            continue
        k0[s // bs, s % bs] = key[i]
        v0[s // bs, s % bs] = value[i]
    assert torch.equal(kc.view(torch.int16), k0.view(torch.int16))
    assert torch.equal(vc.view(torch.int16), v0.view(torch.int16))


# ------------------------------------------------------------------------------ decode

def _scatter_logical(k_log: torch.Tensor, block_table: torch.Tensor, cache: torch.Tensor) -> None:
    """Writes logical tokens k_log [L, Hkv, D] into a paged cache by explicit loop."""
    bs = cache.shape[1]
    for t in range(k_log.shape[0]):
        cache[int(block_table[t // bs]), t % bs] = k_log[t]


def _decode_case(seed, B, hq, hkv, d, bs, max_ctx, nb):
    g = gen(seed)
    ctx = [int(x) for x in torch.randint(1, max_ctx + 1, (B,), generator=g)]
    kc, vc = randn_bf16((nb, bs, hkv, d), g), randn_bf16((nb, bs, hkv, d), g)
    bt = random_block_tables(ctx, bs, nb, g)
    k_log = [randn_bf16((c, hkv, d), g) for c in ctx]
    v_log = [randn_bf16((c, hkv, d), g) for c in ctx]
    for b in range(B):
        _scatter_logical(k_log[b], bt[b], kc)
        _scatter_logical(v_log[b], bt[b], vc)
    q = randn_bf16((B, hq, d), g)
    return q, kc, vc, bt, torch.tensor(ctx, dtype=torch.int32), k_log, v_log


@pytest.mark.parametrize("layout", ["contiguous", "interleaved"])
def test_torch_append_equals_the_byte_level_append(layout):
    """The timed CPU baseline of the append (a torch index-put) writes exactly the bytes
    of the byte-level restatement: valid slots copied, -1 skipped, every other byte of
    the caches (for the page-interleaved pool: of the whole pool) untouched."""
    g = gen(77)
    nb, bs, hkv, d, n = 9, 64, 4, 128, 200
    if layout == "contiguous":
        kc = randn_bf16((nb, bs, hkv, d), g)
        vc = randn_bf16((nb, bs, hkv, d), g)
        base = torch.stack([kc, vc])

        def copies():
            store = base.clone()
            return store[0], store[1], store
    else:
        pool, kc, _ = interleaved_pool(nb, bs, hkv, d, g)

        def copies():  # fresh views into a copy of the pool, with the engine's strides
            store = pool.clone()
            k2, v2 = ref.page_views(store, bs, hkv, d)
            assert k2.stride() == kc.stride()
            return k2, v2, store
    qkv = randn_bf16((n, 3 * hkv * d), g)
    key = randn_bf16((n, hkv, d), g)                                    # contiguous rows
    value = qkv[:, 2 * hkv * d:].view(n, hkv, d)                         # strided rows
    slots = torch.randperm(nb * bs, generator=g)[:n].to(torch.int32)
    slots[::5] = -1
    want_k, want_v, want = copies()
    ref.kv_append(ref.bf16_bits(key), ref.bf16_bits(value.contiguous()), ref.bf16_bits(want_k),
                  ref.bf16_bits(want_v), slots.numpy())
    got_k, got_v, got = copies()
    ref.torch_append(key, value, got_k, got_v, slots)
    assert torch.equal(got.view(torch.uint8), want.view(torch.uint8))
    _, _, before = copies()
    assert not torch.equal(got.view(torch.uint8), before.view(torch.uint8))  # it did write


def test_decode_matches_sdpa_with_gqa():
    """Against torch SDPA(enable_gqa=True) on the logical (unpaged) K/V.  Catches: wrong
    gather through the block table, wrong GQA head map, scale applied twice or not at all."""
    q, kc, vc, bt, ctx, k_log, v_log = _decode_case(3, B=5, hq=8, hkv=2, d=16, bs=4, max_ctx=23, nb=40)
    scale = 0.37
    out = ref.paged_decode(q, kc, vc, bt, ctx, scale, dtype=torch.float64)
    for b in range(q.shape[0]):
        qq = q[b].double().view(1, 8, 1, 16)
        kk = k_log[b].double().transpose(0, 1).unsqueeze(0)
        vv = v_log[b].double().transpose(0, 1).unsqueeze(0)
        want = F.scaled_dot_product_attention(qq, kk, vv, scale=scale, enable_gqa=True)[0, :, 0]
        torch.testing.assert_close(out[b], want, rtol=1e-12, atol=1e-12)


def test_decode_bruteforce_loops():
    """Pure-Python float64 loops over (sequence, head, token) with math.exp, indexing the
    cache through the block table one token at a time."""
    q, kc, vc, bt, ctx, _, _ = _decode_case(4, B=3, hq=4, hkv=2, d=8, bs=4, max_ctx=10, nb=12)
    scale = 0.5
    out = ref.paged_decode(q, kc, vc, bt, ctx, scale, dtype=torch.float64)
    G = 2
    for b in range(3):
        for h in range(4):
            kvh = h // G
            scores = []
            for t in range(int(ctx[b])):
                blk, off = int(bt[b, t // 4]), t % 4
                scores.append(scale * sum(float(q[b, h, e]) * float(kc[blk, off, kvh, e]) for e in range(8)))
            mx = max(scores)
            w = [math.exp(s - mx) for s in scores]
            tot = sum(w)
            for e in range(8):
                val = sum(w[t] * float(vc[int(bt[b, t // 4]), t % 4, kvh, e]) for t in range(len(w))) / tot
                assert abs(val - float(out[b, h, e])) < 1e-12


def test_decode_closed_forms():
    """ctx == 1 returns that token's V (softmax of one score is 1); q == 0 averages V
    over the context; a context of 0 returns zeros."""
    q, kc, vc, bt, _, k_log, v_log = _decode_case(5, B=4, hq=4, hkv=2, d=8, bs=4, max_ctx=9, nb=20)
    one = ref.paged_decode(q, kc, vc, bt, torch.tensor([1, 1, 1, 1]), 0.3, dtype=torch.float64)
    for b in range(4):
        for h in range(4):
            assert torch.equal(one[b, h], v_log[b][0, h // 2].double())
    ctx = torch.tensor([len(v) for v in v_log])
    zero_q = ref.paged_decode(torch.zeros_like(q), kc, vc, bt, ctx, 0.3, dtype=torch.float64)
    for b in range(4):
        for h in range(4):
            torch.testing.assert_close(zero_q[b, h], v_log[b][:, h // 2].double().mean(0), rtol=1e-12, atol=1e-12)
    empty = ref.paged_decode(q, kc, vc, bt, torch.tensor([0, 0, 0, 0]), 0.3)
    assert torch.count_nonzero(empty) == 0


def test_decode_gqa_head_map_and_dominant_key():
    """V constant per kv head: query head h must return the value of kv head h // G
    (catches h % Hkv).  One key scored far above the rest: output is that key's V row
    (catches position <-> physical slot errors)."""
    g = gen(6)
    hq, hkv, d, bs, nb = 8, 4, 8, 4, 8
    kc, vc = randn_bf16((nb, bs, hkv, d), g), torch.zeros(nb, bs, hkv, d, dtype=torch.bfloat16)
    for h in range(hkv):
        vc[:, :, h] = float(h + 1)
    bt = torch.tensor([[3, 6, 1]], dtype=torch.int32)
    q = randn_bf16((1, hq, d), g)
    out = ref.paged_decode(q, kc, vc, bt, torch.tensor([11]), 1.0, dtype=torch.float64)
    for h in range(hq):
        assert torch.allclose(out[0, h], torch.full((d,), float(h // 2 + 1), dtype=torch.float64))
    # dominant key: logical token 6 lives in block bt[1] = 6, offset 2
    vc2 = randn_bf16((nb, bs, hkv, d), g)
    kc2 = torch.zeros(nb, bs, hkv, d, dtype=torch.bfloat16)
    kc2[6, 2] = 8.0
    q2 = torch.ones(1, hq, d, dtype=torch.bfloat16)
    out2 = ref.paged_decode(q2, kc2, vc2, bt, torch.tensor([11]), 1.0, dtype=torch.float64)
    for h in range(hq):
        torch.testing.assert_close(out2[0, h], vc2[6, 2, h // 2].double(), rtol=0, atol=1e-9)


def test_decode_block_renumbering_invariant():
    """Moving blocks to other physical ids (and rewriting the table) changes nothing."""
    q, kc, vc, bt, ctx, _, _ = _decode_case(7, B=4, hq=4, hkv=1, d=8, bs=4, max_ctx=15, nb=24)
    out = ref.paged_decode(q, kc, vc, bt, ctx, 0.4, dtype=torch.float64)
    perm = torch.randperm(24, generator=gen(70))
    kc2, vc2 = torch.empty_like(kc), torch.empty_like(vc)
    kc2[perm] = kc
    vc2[perm] = vc
    bt2 = torch.where(bt >= 0, perm[bt.clamp(min=0).long()].to(torch.int32), bt)
    out2 = ref.paged_decode(q, kc2, vc2, bt2, ctx, 0.4, dtype=torch.float64)
    assert torch.equal(out, out2)


# ------------------------------------------------------------------------------ prefill

def _sdpa(q, k, v, scale, mask=None, causal=False):
    return F.scaled_dot_product_attention(q, k, v, attn_mask=mask, is_causal=causal,
                                          scale=scale, enable_gqa=True)


def test_prefill_equal_lengths_is_standard_causal():
    """klen == qlen: bottom-right and top-left alignment coincide, so the oracle must equal
    SDPA(is_causal=True) per sequence."""
    g = gen(8)
    lens = [5, 1, 12]
    hq, hkv, d = 4, 2, 16
    T = sum(lens)
    q, k, v = randn_bf16((T, hq, d), g), randn_bf16((T, hkv, d), g), randn_bf16((T, hkv, d), g)
    cu = torch.tensor([0, 5, 6, 18], dtype=torch.int32)
    out = ref.varlen_prefill(q, k, v, cu, cu, 0.25, dtype=torch.float64)
    for s in range(3):
        a, b = int(cu[s]), int(cu[s + 1])
        want = _sdpa(q[a:b].double().transpose(0, 1), k[a:b].double().transpose(0, 1),
                     v[a:b].double().transpose(0, 1), 0.25, causal=True).transpose(0, 1)
        torch.testing.assert_close(out[a:b], want, rtol=1e-12, atol=1e-12)


def test_prefill_bottom_right_alignment():
    """qlen < klen (cached prefix): the last query sees every key, the first query sees
    keys 0..klen-qlen.  A top-left mask fails both."""
    g = gen(9)
    qlen, klen, hq, hkv, d = 4, 11, 2, 1, 8
    q = randn_bf16((qlen, hq, d), g)
    k, v = randn_bf16((klen, hkv, d), g), randn_bf16((klen, hkv, d), g)
    out = ref.varlen_prefill(q, k, v, torch.tensor([0, qlen]), torch.tensor([0, klen]), 0.5,
                             dtype=torch.float64)
    qq, kk, vv = (x.double().transpose(0, 1) for x in (q, k, v))
    last = _sdpa(qq[:, -1:], kk, vv, 0.5).transpose(0, 1)[0]
    first = _sdpa(qq[:, :1], kk[:, :klen - qlen + 1], vv[:, :klen - qlen + 1], 0.5).transpose(0, 1)[0]
    torch.testing.assert_close(out[-1], last, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(out[0], first, rtol=1e-12, atol=1e-12)


def test_prefill_paged_equals_dense_and_noncausal_is_full():
    """Paged mode on scattered blocks equals dense mode on the packed rows; causal=False
    equals unmasked SDPA."""
    g = gen(10)
    hq, hkv, d, bs, nb = 4, 2, 8, 4, 30
    qlens, klens = [3, 6, 1], [9, 6, 5]
    q = randn_bf16((sum(qlens), hq, d), g)
    kd, vd = randn_bf16((sum(klens), hkv, d), g), randn_bf16((sum(klens), hkv, d), g)
    cq = torch.tensor(np.cumsum([0] + qlens), dtype=torch.int32)
    ck = torch.tensor(np.cumsum([0] + klens), dtype=torch.int32)
    kc, vc = randn_bf16((nb, bs, hkv, d), g), randn_bf16((nb, bs, hkv, d), g)
    bt = random_block_tables(klens, bs, nb, g)
    for s in range(3):
        _scatter_logical(kd[ck[s]:ck[s + 1]], bt[s], kc)
        _scatter_logical(vd[ck[s]:ck[s + 1]], bt[s], vc)
    dense = ref.varlen_prefill(q, kd, vd, cq, ck, 0.3, dtype=torch.float64)
    paged = ref.varlen_prefill(q, kc, vc, cq, ck, 0.3, block_tables=bt, dtype=torch.float64)
    assert torch.equal(dense, paged)
    full = ref.varlen_prefill(q, kd, vd, cq, ck, 0.3, causal=False, dtype=torch.float64)
    for s in range(3):
        qq = q[cq[s]:cq[s + 1]].double().transpose(0, 1)
        kk = kd[ck[s]:ck[s + 1]].double().transpose(0, 1)
        vv = vd[ck[s]:ck[s + 1]].double().transpose(0, 1)
        torch.testing.assert_close(full[cq[s]:cq[s + 1]], _sdpa(qq, kk, vv, 0.3).transpose(0, 1),
                                   rtol=1e-12, atol=1e-12)


def test_prefill_rows_without_keys_are_zero():
    """klen < qlen leaves the first qlen-klen rows with no visible key: zeros."""
    g = gen(11)
    q = randn_bf16((5, 2, 8), g)
    k, v = randn_bf16((3, 1, 8), g), randn_bf16((3, 1, 8), g)
    out = ref.varlen_prefill(q, k, v, torch.tensor([0, 5]), torch.tensor([0, 3]), 1.0)
    assert torch.count_nonzero(out[:2]) == 0 and torch.count_nonzero(out[2:]) > 0


# ------------------------------------------------------------------------------ metadata

def test_prefill_metadata_known_answer():
    """Hand-worked case: blocks [7, 3], 2 cached tokens, 4 new, block size 4: positions
    2..5 go to slots 30, 31 (block 7) and 12, 13 (block 3); block tables are emitted
    because cu_seqlens_k (6) exceeds cu_seqlens_q (4)."""
    m = ref.prefill_metadata([[7, 3]], [2], [4], 4)
    assert m["slot_mapping"] == [30, 31, 12, 13]
    assert m["positions"] == [2, 3, 4, 5]
    assert m["cu_seqlens_q"] == [0, 4] and m["cu_seqlens_k"] == [0, 6]
    assert m["block_tables"] == [[7, 3]]
    m2 = ref.prefill_metadata([[1], [4, 2]], [0, 0], [3, 6], 4)
    assert m2["block_tables"] is None and m2["slot_mapping"] == [4, 5, 6, 16, 17, 18, 19, 8, 9]


def test_prefill_metadata_matches_block_range_construction():
    """The reference builds slots block range by block range (model_runner.py:420-430);
    that construction, restated here, must agree with the per-position formula."""
    rng = np.random.default_rng(12)
    bs = 8
    for _ in range(50):
        n_seq = rng.integers(1, 5)
        tables, cached, sched = [], [], []
        for _ in range(n_seq):
            total = int(rng.integers(1, 60))
            c = int(rng.integers(0, total))
            tables.append([int(x) for x in rng.permutation(200)[:math.ceil(total / bs)]])
            cached.append(c)
            sched.append(total - c)
        want = []
        for bt, start, n in zip(tables, cached, sched):
            end = start + n
            sb, eb = start // bs, (end + bs - 1) // bs
            for i in range(sb, eb):
                lo = bt[i] * bs + (start % bs if i == sb else 0)
                hi = bt[i] * bs + (bs if i != eb - 1 else end - i * bs)
                want.extend(range(lo, hi))
        assert ref.prefill_metadata(tables, cached, sched, bs)["slot_mapping"] == want


def test_decode_metadata_last_slot_and_padding():
    """Decode slot from the last-block formula equals block_table[pos // bs] * bs + pos % bs
    for pos = len - 1; rows are padded with -1."""
    m = ref.decode_metadata([[5, 9], [2]], [6, 3], 4)
    assert m["slot_mapping"] == [37, 10] and m["context_lens"] == [6, 3]
    assert m["positions"] == [5, 2] and m["block_tables"] == [[5, 9], [2, -1]]
    rng = np.random.default_rng(13)
    for _ in range(100):
        n = int(rng.integers(1, 100))
        bt = [int(x) for x in rng.permutation(500)[:math.ceil(n / 16)]]
        slot = ref.decode_metadata([bt], [n], 16)["slot_mapping"][0]
        assert slot == bt[(n - 1) // 16] * 16 + (n - 1) % 16


def test_traffic_and_flop_counts():
    """Known answers for the algorithmic byte / flop counts used in the roofline."""
    # ctx 1, 256, 257 with Hq 2, Hkv 1, D 4, bs 256:
    # KV 514 tokens * 4 dims * 2 B * 2 tensors, q+o 3*2*4*2*2, lens 12 B, table entries 4*4 B
    assert ref.decode_bytes([1, 256, 257], 2, 1, 4, 256) == 8224 + 96 + 12 + 16
    assert ref.append_bytes([3, -1, 9], 8, 128) == 2 * 8 * 128 * 2 * 4 + 12
    # qlen 2, klen 3 causal: query 0 sees keys 0..1, query 1 sees 0..2 -> 5 pairs
    assert ref.prefill_flops([0, 2], [0, 3], 1, 1) == 4 * 5
    assert ref.prefill_flops([0, 2], [0, 3], 2, 8, causal=False) == 4 * 2 * 8 * 6


def test_cpu_baselines_agree_with_oracle():
    """The timed bf16 SDPA baselines compute the same function as the oracle."""
    q, kc, vc, bt, ctx, _, _ = _decode_case(14, B=3, hq=4, hkv=2, d=16, bs=4, max_ctx=14, nb=16)
    got = ref.sdpa_paged_decode(q, kc, vc, bt, ctx, 0.25).float()
    torch.testing.assert_close(got, ref.paged_decode(q, kc, vc, bt, ctx, 0.25), atol=2e-2, rtol=1e-2)
    g = gen(15)
    q2 = randn_bf16((7, 4, 16), g)
    k2, v2 = randn_bf16((10, 2, 16), g), randn_bf16((10, 2, 16), g)
    cq, ck = torch.tensor([0, 3, 7]), torch.tensor([0, 4, 10])
    got2 = ref.sdpa_varlen_prefill(q2, k2, v2, cq, ck, 0.25).float()
    torch.testing.assert_close(got2, ref.varlen_prefill(q2, k2, v2, cq, ck, 0.25), atol=2e-2, rtol=1e-2)
