"""Fused layer kernels (RMSNorm, q/k norm + RoPE + append, SiLU * up, argmax) against
the layer oracle, on the GPU.

The cases restate the reference's tests/test_fused_kernels.py:40-100 (same shapes,
strided q/k views, a non-power-of-two head size, rtol = atol = 2e-2, greedy == argmax on
[512, 151936]) and add what the fused append must keep bit-exact: v copied bit for bit,
-1 and out-of-range slots skipped, untouched slots unchanged, K/V-interleaved pages.
"""

import pytest
import torch

from kavor_amd.layers.fused import add_rms_norm, greedy_argmax, qk_norm_rope_append, rms_norm, silu_and_mul
from oracle import layers_oracle as ref
from oracle.kvpath_oracle import page_views

pytestmark = pytest.mark.gpu
EPS = 1e-6
TOL = dict(rtol=2e-2, atol=2e-2)


def _randn(*shape, gen, scale=1.0):
    return (torch.randn(*shape, generator=gen) * scale).to(torch.bfloat16)


@pytest.mark.parametrize("shape,view", [
    ((128, 4096), False), ((1, 4096), False), ((300, 1024), False), ((7, 2048), False),
    ((3, 8192), False), ((9, 136), False), ((37, 32, 128), True), ((5, 8, 80), True),
])
def test_rmsnorm_matches_oracle(cuda_device, shape, view):
    g = torch.Generator().manual_seed(0)
    w = _randn(shape[-1], gen=g)
    if view:
        buf = _randn(shape[0], shape[1] * 3, shape[2], gen=g)
        x = buf[:, :shape[1], :]
    else:
        x = _randn(*shape, gen=g)
    want = ref.rms_norm(x, w, EPS).float()
    got = rms_norm(x.to(cuda_device), w.to(cuda_device), EPS)
    torch.testing.assert_close(got.cpu().float(), want, **TOL)


@pytest.mark.parametrize("rows,cols", [(256, 4096), (256, 1024), (1, 1024), (4099, 1024)])
def test_add_rmsnorm_matches_oracle(cuda_device, rows, cols):
    g = torch.Generator().manual_seed(1)
    x, r, w = _randn(rows, cols, gen=g), _randn(rows, cols, gen=g), _randn(cols, gen=g)
    want, want_res = ref.add_rms_norm(x, r, w, EPS)
    res_dev = r.to(cuda_device)
    got, res = add_rms_norm(x.to(cuda_device), res_dev, w.to(cuda_device), EPS)
    assert res.data_ptr() == res_dev.data_ptr()          # updated in place
    assert torch.equal(res.cpu(), want_res)              # bf16(x + r): exact
    torch.testing.assert_close(got.cpu().float(), want.float(), **TOL)


def _pool(num_blocks, bs, hkv, D, dev, gen):
    page = 2 * bs * hkv * D * 2
    raw = torch.randint(0, 256, (num_blocks, page), generator=gen, dtype=torch.uint8)
    pool = raw.to(dev)
    return raw, pool, page_views(pool, bs, hkv, D)


@pytest.mark.parametrize("T,hq,hkv", [(64, 32, 8), (300, 16, 8), (5, 16, 16), (1, 16, 8),
                                      (3, 5, 1), (2048, 16, 8), (2050, 32, 8), (2050, 40, 8),
                                      (2049, 5, 1)])
def test_qk_norm_rope_append(cuda_device, T, hq, hkv):
    """A token's hq + 2*hkv head rows are cut into groups, one wave per group, each of the
    wave's four 16-lane rows taking NB head rows: below 2048 tokens NB = 1 (groups of 4
    rows), from 2048 on NB = 4 (groups of 16).  (3, 5, 1) has 7 rows, so its second
    group of 4 has one idle row; (2050, 40, 8) has 56 rows, so the fourth group of 16 has
    8 idle rows; (2049, 5, 1) fits in one group of 16 with 9 idle.  The idle rows load a
    clamped head and store nothing."""
    D, bs, nb, max_pos = 128, 64, 40, 4096
    g = torch.Generator().manual_seed(2)
    qkv = _randn(T, (hq + 2 * hkv) * D, gen=g)
    pos = torch.randint(0, max_pos, (T,), generator=g, dtype=torch.int32)
    table = ref.rope_table(D, max_pos, 1e6)
    qw, kw = _randn(D, gen=g), _randn(D, gen=g)
    slots = torch.randperm(nb * bs, generator=g)[:T].to(torch.int32)
    slots[::7] = -1
    slots[3 % T] = nb * bs + 5                          # out of range: skipped
    raw, pool, (kc, vc) = _pool(nb, bs, hkv, D, cuda_device, g)
    q = qk_norm_rope_append(qkv.to(cuda_device), pos.to(cuda_device), table.to(cuda_device),
                            qw.to(cuda_device), kw.to(cuda_device), EPS, hq, hkv,
                            kc, vc, slots.to(cuda_device))
    wq, wk, wv = ref.qk_norm_rope(qkv, pos, table, qw, kw, EPS, hq, hkv)
    torch.testing.assert_close(q.cpu().float(), wq.float(), **TOL)

    kc_h, vc_h = page_views(pool.cpu(), bs, hkv, D)
    want_k, want_v = page_views(raw.clone(), bs, hkv, D)
    valid = [(i, int(s)) for i, s in enumerate(slots) if 0 <= s < nb * bs]
    for i, s in valid:
        want_k[s // bs, s % bs] = wk[i]
        want_v[s // bs, s % bs] = wv[i]
    # v and every untouched byte are exact; k within the RoPE tolerance
    assert torch.equal(vc_h.view(torch.int16), want_v.view(torch.int16))
    mask = torch.zeros(nb, bs, dtype=torch.bool)
    for _, s in valid:
        mask[s // bs, s % bs] = True
    assert torch.equal(kc_h[~mask].view(torch.int16), want_k[~mask].view(torch.int16))
    torch.testing.assert_close(kc_h[mask].float(), want_k[mask].float(), **TOL)


@pytest.mark.parametrize("T,hq,hkv", [(1, 16, 8), (300, 16, 8), (2050, 32, 8), (7, 5, 1)])
def test_qk_norm_rope_k_out(cuda_device, T, hq, hkv):
    """The no-append variant: q and k come out as fresh tensors (k contiguous, Hkv heads),
    v is not read (NaN-filled v heads must not leak), and nothing else is written."""
    from kavor_amd.layers.fused import qk_norm_rope

    D, max_pos = 128, 4096
    g = torch.Generator().manual_seed(12)
    qkv = _randn(T, (hq + 2 * hkv) * D, gen=g)
    qkv[:, (hq + hkv) * D:] = float("nan")
    pos = torch.randint(0, max_pos, (T,), generator=g, dtype=torch.int32)
    table = ref.rope_table(D, max_pos, 1e6)
    qw, kw = _randn(D, gen=g), _randn(D, gen=g)
    q, k = qk_norm_rope(qkv.to(cuda_device), pos.to(cuda_device), table.to(cuda_device),
                        qw.to(cuda_device), kw.to(cuda_device), EPS, hq, hkv)
    wq, wk, _ = ref.qk_norm_rope(qkv, pos, table, qw, kw, EPS, hq, hkv)
    assert q.shape == (T, hq, D) and k.shape == (T, hkv, D) and k.is_contiguous()
    torch.testing.assert_close(q.cpu().float(), wq.float(), **TOL)
    torch.testing.assert_close(k.cpu().float(), wk.float(), **TOL)
    # the same kernel with the append writes the same k bits into the pages
    bs, nb = 64, -(-T // 64) + 1
    raw, pool, (kc, vc) = _pool(nb, bs, hkv, D, cuda_device, g)
    slots = torch.arange(T, dtype=torch.int32)
    q2 = qk_norm_rope_append(qkv.to(cuda_device), pos.to(cuda_device), table.to(cuda_device),
                             qw.to(cuda_device), kw.to(cuda_device), EPS, hq, hkv, kc, vc, slots.to(cuda_device))
    torch.cuda.synchronize()
    assert torch.equal(q2.cpu().view(torch.int16), q.cpu().view(torch.int16))
    got_k = kc.reshape(nb * bs, hkv, D)[:T].cpu()
    assert torch.equal(got_k.view(torch.int16), k.cpu().view(torch.int16))


def test_qk_norm_rope_without_append_and_bad_position(cuda_device):
    D, hq, hkv, T = 128, 16, 8, 4
    g = torch.Generator().manual_seed(3)
    qkv = _randn(T, (hq + 2 * hkv) * D, gen=g)
    table = ref.rope_table(D, 100, 1e6)
    ones = torch.ones(D, dtype=torch.bfloat16)
    pos = torch.tensor([0, 99, 100, 5], dtype=torch.int32)     # 100 is out of range
    q = qk_norm_rope_append(qkv.to(cuda_device), pos.to(cuda_device), table.to(cuda_device),
                            ones.to(cuda_device), ones.to(cuda_device), EPS, hq, hkv, None, None, None).cpu()
    assert torch.isnan(q[2].float()).all() and torch.isfinite(q[[0, 1, 3]].float()).all()
    wq, _, _ = ref.qk_norm_rope(qkv, pos.clamp(max=99), table, ones, ones, EPS, hq, hkv)
    torch.testing.assert_close(q[[0, 1, 3]].float(), wq[[0, 1, 3]].float(), **TOL)


@pytest.mark.parametrize("T,I", [(256, 3072), (1, 3072), (1000, 1024), (3, 8)])
def test_silu_and_mul(cuda_device, T, I):
    g = torch.Generator().manual_seed(4)
    gu = _randn(T, 2 * I, gen=g, scale=3.0)
    got = silu_and_mul(gu.to(cuda_device)).cpu()
    torch.testing.assert_close(got.float(), ref.silu_and_mul(gu).float(), **TOL)


def test_greedy_argmax_matches_torch(cuda_device):
    g = torch.Generator().manual_seed(5)
    logits = (torch.randn(512, 151936, generator=g) * 3).to(torch.bfloat16)
    logits[7, 100] = logits[7, 90000] = 50.0          # tie: first index wins
    logits[9, :] = 1.0                                 # all equal: index 0
    logits[11, 151935] = 60.0                          # last element
    got = greedy_argmax(logits.to(cuda_device)).cpu()
    assert got.dtype == torch.int64
    assert torch.equal(got, ref.greedy(logits))
    assert got[7].item() == 100 and got[9].item() == 0 and got[11].item() == 151935


def test_greedy_argmax_odd_vocab_and_nan(cuda_device):
    g = torch.Generator().manual_seed(6)
    logits = _randn(3, 1003, gen=g)
    logits[0, 1001] = 40.0                             # in the scalar tail
    logits[1, 17] = float("nan")
    logits[1, 500] = float("nan")
    buf = torch.zeros(3, 1008, dtype=torch.bfloat16)
    buf[:, :1003] = logits                             # row stride 1008, vocab 1003
    got = greedy_argmax(buf.to(cuda_device)[:, :1003]).cpu()
    assert got.tolist() == [1001, 17, int(logits[2].float().argmax())]


def test_greedy_argmax_screen_edge_cases(cuda_device):
    """Rows that the per-chunk screen (max tree + NaN-probing sum) must hand to the exact
    comparison: all -inf, signed zeros tied, +inf and -inf in one chunk, a negative NaN,
    NaN after +inf; and a vocabulary that needs a second round of loads."""
    V = 200_000  # 25,000 chunks: past one round of 1024 threads x 20 loads
    rows = torch.full((8, V), -1.0).to(torch.bfloat16)
    rows[0, :] = float("-inf")                               # all -inf: index 0
    rows[1, 3], rows[1, 5] = -0.0, 0.0                       # -0 == +0: first index
    rows[2, 3], rows[2, 5] = 0.0, -0.0
    rows[3, 8], rows[3, 9], rows[3, 77_777] = float("inf"), float("-inf"), 5.0   # +inf wins
    rows[4, 40] = 2.0
    rows[4].view(torch.int16)[60_000] = -64                  # 0xFFC0: a negative quiet NaN
    rows[5, 10], rows[5, 190_000] = float("inf"), float("nan")  # NaN above +inf
    rows[6, 170_001] = 9.0                                   # only in the second round
    rows[7, 100] = 3.0
    rows[7, 180_000] = 3.0                                   # tie across rounds: first
    got = greedy_argmax(rows.to(cuda_device)).cpu()
    assert got.tolist() == [0, 3, 3, 8, 60_000, 190_000, 170_001, 100]
    assert torch.equal(got, ref.greedy(rows))


@pytest.mark.parametrize("rows", [1, 7, 100, 191, 192])
def test_greedy_argmax_split_rows_equal_whole_rows(cuda_device, rows):
    """Below 192 rows each row is split over several workgroups (up to 16 segments) whose
    best (value, index) pairs are merged as ordered 64-bit keys.  The result must equal
    the whole-row kernel (no workspace) and torch.argmax, with ties and NaNs placed
    across segment boundaries and in the tail."""
    from kavor_amd._lib import check, lib

    V = 151936 + 5
    g = torch.Generator().manual_seed(40 + rows)
    logits = (torch.randn(rows, V, generator=g) * 3).to(torch.bfloat16)
    logits[0, 9000] = logits[0, 150000] = 70.0          # tie across segments: first wins
    if rows > 1:
        logits[1, 151937] = 80.0                         # in the scalar tail
    if rows > 2:
        logits[2, 4] = float("nan")
        logits[2, 120000] = float("nan")                 # first NaN wins
        logits[3 % rows, :] = -0.0
        logits[3 % rows, 60000] = 0.0                    # -0 == +0: index 0 wins
    buf = torch.zeros(rows, V + 3, dtype=torch.bfloat16)
    buf[:, :V] = logits
    dev_logits = buf.to(cuda_device)[:, :V]
    split = greedy_argmax(dev_logits).cpu()
    whole = torch.empty(rows, dtype=torch.int64, device=cuda_device)
    rc = lib().kvp_argmax_bf16(dev_logits.data_ptr(), dev_logits.stride(0), rows, V, whole.data_ptr(),
                               None, 0, torch.cuda.current_stream(cuda_device).cuda_stream)
    check("kvp_argmax_bf16", rc)
    assert torch.equal(split, whole.cpu())
    assert torch.equal(split, ref.greedy(logits))
    assert split[0].item() == 9000


@pytest.mark.parametrize("vocab", [1, 5, 8, 13])
def test_greedy_argmax_tiny_vocab(cuda_device, vocab):
    g = torch.Generator().manual_seed(7 + vocab)
    logits = _randn(4, vocab, gen=g)
    logits[1, vocab - 1] = 30.0
    buf = torch.zeros(4, 16, dtype=torch.bfloat16)  # row stride: a multiple of 8 elements
    buf[:, :vocab] = logits
    got = greedy_argmax(buf.to(cuda_device)[:, :vocab]).cpu()
    assert torch.equal(got, ref.greedy(logits))
    assert got[1].item() == vocab - 1
