"""GPU parity of paged decode (kvp_paged_decode_bf16 via kavor_amd.layers.attention.paged_decode)
against the fp32 oracle, within atol 2e-2 / rtol 1e-2 on the bf16 output."""

import math

import numpy as np
import pytest
import torch

from oracle import kvpath_oracle as ref
from tests.helpers import (TOL, gen, randn_bf16, interleaved_pool, contiguous_caches, random_block_tables,
                           bits_equal, relocate_pages)
from tests.test_golden import load, bf16

pytestmark = pytest.mark.gpu
SCALE = 128 ** -0.5


def _decode(q, kc, vc, ctx, bt, scale=SCALE, **kw):
    from kavor_amd.layers.attention import paged_decode

    return paged_decode(q, kc, vc, cache_seqlens=ctx, block_table=bt, softmax_scale=scale, **kw)


def _case(seed, B, hq, hkv, bs, lo, hi, nb=None, layout="contiguous", width=None):
    g = gen(seed)
    ctx = torch.randint(lo, hi + 1, (B,), generator=g, dtype=torch.int32)
    need = sum(math.ceil(int(c) / bs) for c in ctx)
    nb = nb or need + 3
    if layout == "contiguous":
        kc, vc = contiguous_caches(nb, bs, hkv, 128, g)
    else:
        _, kc, vc = interleaved_pool(nb, bs, hkv, 128, g)
    bt = random_block_tables([int(c) for c in ctx], bs, nb, g, width=width)
    q = randn_bf16((B, hq, 128), g)
    return q, kc, vc, bt, ctx


def _check(dev, q, kc, vc, bt, ctx, tol=TOL):
    out = _decode(q.to(dev), kc.to(dev), vc.to(dev), ctx.to(dev), bt.to(dev))
    torch.cuda.synchronize()
    want = ref.paged_decode(q, kc, vc, bt, ctx, SCALE)
    torch.testing.assert_close(out.cpu().float(), want, **tol)
    return out


@pytest.mark.parametrize("G", [1, 2, 4, 5, 8])
@pytest.mark.parametrize("bs,layout", [(256, "interleaved"), (64, "contiguous"), (128, "interleaved")])
def test_decode_matches_oracle(cuda_device, G, bs, layout):
    hkv = 2
    q, kc, vc, bt, ctx = _case(10 * G + bs, B=12, hq=G * hkv, hkv=hkv, bs=bs, lo=1, hi=1500, layout=layout)
    _check(cuda_device, q, kc, vc, bt, ctx)


def test_decode_4d_query_and_out_buffer(cuda_device):
    """q given as [B, 1, Hq, D] (the reference's q.unsqueeze(1)) returns [B, 1, Hq, D]; a
    preallocated, strided out buffer is honoured."""
    q, kc, vc, bt, ctx = _case(11, B=5, hq=16, hkv=8, bs=256, lo=1, hi=700)
    d = cuda_device
    out4 = _decode(q.to(d).unsqueeze(1), kc.to(d), vc.to(d), ctx.to(d), bt.to(d))
    assert out4.shape == (5, 1, 16, 128)
    big = torch.full((5, 20, 128), 7.0, dtype=torch.bfloat16, device=d)
    _decode(q.to(d), kc.to(d), vc.to(d), ctx.to(d), bt.to(d), out=big[:, 2:18])
    torch.cuda.synchronize()
    assert bits_equal(big[:, 2:18].cpu(), out4[:, 0].cpu())
    assert torch.all(big[:, :2] == 7.0) and torch.all(big[:, 18:] == 7.0)


def test_decode_context_edges(cuda_device):
    """ctx 0 -> zeros, ctx 1 -> that token's V row exactly, block-boundary lengths."""
    q, kc, vc, bt, _ = _case(12, B=8, hq=16, hkv=8, bs=256, lo=513, hi=513)
    ctx = torch.tensor([0, 1, 255, 256, 257, 511, 512, 513], dtype=torch.int32)
    out = _check(cuda_device, q, kc, vc, bt, ctx).cpu()
    assert torch.count_nonzero(out[0]) == 0
    for h in range(16):
        assert bits_equal(out[1, h], vc[int(bt[1, 0]), 0, h // 2])


def test_decode_stale_table_columns_are_not_read(cuda_device):
    """Graph replay leaves stale block ids past ceil(ctx/bs) (model_runner.py:235); eager
    pads with -1.  Both, and out-of-range garbage, give identical results."""
    q, kc, vc, bt, ctx = _case(13, B=16, hq=16, hkv=8, bs=64, lo=1, hi=900, width=20)
    d = cuda_device
    base = _decode(q.to(d), kc.to(d), vc.to(d), ctx.to(d), bt.to(d)).cpu()
    junk = bt.clone()
    junk[junk < 0] = torch.randint(-(1 << 30), 1 << 30, (int((junk < 0).sum()),), generator=gen(130), dtype=torch.int32)
    got = _decode(q.to(d), kc.to(d), vc.to(d), ctx.to(d), junk.to(d)).cpu()
    assert bits_equal(base, got)


def test_decode_invalid_block_poisons_only_its_sequence(cuda_device):
    q, kc, vc, bt, ctx = _case(14, B=6, hq=16, hkv=8, bs=256, lo=300, hi=900)
    nb = kc.shape[0]
    bad = bt.clone()
    bad[2, 1] = nb + 5      # needed block beyond the pool
    bad[4, 0] = -3          # negative id
    d = cuda_device
    out = _decode(q.to(d), kc.to(d), vc.to(d), ctx.to(d), bad.to(d)).cpu().float()
    assert torch.isnan(out[2]).all() and torch.isnan(out[4]).all()
    good = [0, 1, 3, 5]
    want = ref.paged_decode(q[good], kc, vc, bt[good], ctx[good], SCALE)
    torch.testing.assert_close(out[good], want, **TOL)
    over = ctx.clone()
    over[0] = bt.shape[1] * 256 + 1   # longer than the table can describe
    out2 = _decode(q.to(d), kc.to(d), vc.to(d), over.to(d), bt.to(d)).cpu().float()
    assert torch.isnan(out2[0]).all() and not torch.isnan(out2[1:]).any()


def test_decode_deterministic_and_permutation_consistent(cuda_device):
    """Repeating a call gives identical bits.  Permuting the batch moves the points where
    the work split cuts a sequence (the split balances the whole batch), so the permuted
    outputs agree within tolerance, and both agree with the oracle."""
    q, kc, vc, bt, ctx = _case(15, B=32, hq=16, hkv=8, bs=256, lo=1, hi=2048)
    d = cuda_device
    perm = torch.randperm(32, generator=gen(150))
    a = _decode(q.to(d), kc.to(d), vc.to(d), ctx.to(d), bt.to(d)).cpu()
    a2 = _decode(q.to(d), kc.to(d), vc.to(d), ctx.to(d), bt.to(d)).cpu()
    assert bits_equal(a, a2)
    b = _decode(q[perm].to(d), kc.to(d), vc.to(d), ctx[perm].to(d), bt[perm].contiguous().to(d)).cpu()
    torch.testing.assert_close(a[perm].float(), b.float(), **TOL)
    torch.testing.assert_close(a.float(), ref.paged_decode(q, kc, vc, bt, ctx, SCALE), **TOL)


def test_decode_table_width_stays_within_tolerance(cuda_device):
    """The block-table width sizes the work split (and the workspace); a wider table
    changes how many partial states the same sequences produce.  Both agree with the
    oracle."""
    q, kc, vc, bt, ctx = _case(16, B=8, hq=32, hkv=8, bs=256, lo=2000, hi=8192, width=40)
    d = cuda_device
    wide = _decode(q.to(d), kc.to(d), vc.to(d), ctx.to(d), bt.to(d)).cpu().float()
    narrow = _decode(q.to(d), kc.to(d), vc.to(d), ctx.to(d), bt[:, :32].contiguous().to(d)).cpu().float()
    want = ref.paged_decode(q, kc, vc, bt, ctx, SCALE)
    torch.testing.assert_close(wide, want, **TOL)
    torch.testing.assert_close(narrow, want, **TOL)


def test_decode_graph_replay_matches_eager(cuda_device):
    """Capture with zero metadata (as capture_cudagraph does), then replay with new
    lengths and tables: every replay equals the eager call bit for bit."""
    B, hq, hkv, bs, width = 16, 16, 8, 256, 16
    g = gen(17)
    nb = 300
    d = cuda_device
    kc, vc = (t.to(d) for t in contiguous_caches(nb, bs, hkv, 128, g))
    q = randn_bf16((B, hq, 128), g).to(d)
    ctx_buf = torch.zeros(B, dtype=torch.int32, device=d)
    bt_buf = torch.zeros(B, width, dtype=torch.int32, device=d)
    out = _decode(q, kc, vc, ctx_buf, bt_buf)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _decode(q, kc, vc, ctx_buf, bt_buf, out=out)
    for step in range(3):
        gs = gen(170 + step)
        ctx = torch.randint(0, 4096, (B,), generator=gs, dtype=torch.int32)
        bt = random_block_tables([int(c) for c in ctx], bs, nb, gs, width=width, pad=7)
        ctx_buf.copy_(ctx.to(d))
        bt_buf.copy_(bt.to(d))
        graph.replay()
        torch.cuda.synchronize()
        replay = out.clone()
        eager = _decode(q, kc, vc, ctx_buf, bt_buf)
        torch.cuda.synchronize()
        assert bits_equal(replay, eager)
    torch.testing.assert_close(replay.cpu().float(), ref.paged_decode(q.cpu(), kc.cpu(), vc.cpu(), bt, ctx, SCALE), **TOL)



def test_graph_keeps_its_workspace_when_an_eager_call_grows_it(cuda_device):
    """A graph captured with the workspace reserved for its batch keeps launching on that
    buffer after an eager call with a larger batch has grown the workspace.  The old
    buffer must stay allocated: a tensor allocated after the growth (which the caching
    allocator would place in a freed block of that size) is never written by a replay."""
    from kavor_amd.layers import attention

    d = cuda_device
    B, hq, hkv, bs, width, nb = 8, 16, 8, 256, 16, 300
    g = gen(23)
    kc, vc = (t.to(d) for t in contiguous_caches(nb, bs, hkv, 128, g))
    q = randn_bf16((B, hq, 128), g).to(d)
    ctx = torch.randint(3000, 4096, (B,), generator=g, dtype=torch.int32)
    bt = random_block_tables([int(c) for c in ctx], bs, nb, g, width=width)
    ctx_d, bt_d = ctx.to(d), bt.to(d)
    ws = attention._workspaces.pop(d.index, None)  # start from a workspace sized for this batch
    if ws is not None:  # graphs captured earlier in this process may still use it
        attention._retired_workspaces.append(ws)
    attention.reserve_decode_workspace(B, hq, 128, width, bs, d)
    old_bytes = attention._workspaces[d.index].numel()
    out = _decode(q, kc, vc, ctx_d, bt_d)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _decode(q, kc, vc, ctx_d, bt_d, out=out)
    qb = randn_bf16((8 * B, hq, 128), g).to(d)
    ctx_b = ctx.repeat(8).to(d)
    bt_b = bt.repeat(8, 1).to(d)
    _decode(qb, kc, vc, ctx_b, bt_b)  # grows the workspace
    assert attention._workspaces[d.index].numel() > old_bytes
    junk = torch.full((old_bytes,), 0x5A, dtype=torch.uint8, device=d)
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    assert bool((junk == 0x5A).all())
    assert bits_equal(out, _decode(q, kc, vc, ctx_d, bt_d))

def _device_oracle_check(q, kc, vc, bt, ctx, out, chunk=32):
    """Every sequence of a full-size run against the fp32 oracle, evaluated on the
    device in float32 (full-precision matmuls), a chunk of sequences at a time."""
    allow = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        for b0 in range(0, q.shape[0], chunk):
            sl = slice(b0, b0 + chunk)
            want = ref.paged_decode(q[sl], kc, vc, bt[sl], ctx[sl], SCALE)
            torch.testing.assert_close(out[sl].float(), want, **TOL, msg=lambda m: f"sequences {b0}+: {m}")
    finally:
        torch.backends.cuda.matmul.allow_tf32 = allow


@pytest.mark.parametrize("shape", ["qwen3_0.6b", "qwen3_8b"])
def test_decode_full_size_every_sequence(cuda_device, shape):
    """The two decode workloads at full size: Qwen3-0.6B (B=256, 16q/8kv, ctx 100-2048,
    4096-block pool) and Qwen3-8B (B=128, 32q/8kv, ctx 1024-32768, 20000-block pool).
    Every sequence is compared with the fp32 oracle, so a fault in the stream-K split
    that hits only some sequences of the real batch (a range cut at the wrong step, a
    step dealt twice, a merge slot off by one) fails here."""
    B, hq, lo, hi, nb = (256, 16, 100, 2048, 4096) if shape == "qwen3_0.6b" else (128, 32, 1024, 32768, 20000)
    hkv, bs, d = 8, 256, cuda_device
    g = gen(18)
    ctx = torch.randint(lo, hi + 1, (B,), generator=g, dtype=torch.int32)
    bt = random_block_tables([int(c) for c in ctx], bs, nb, g)
    dg = torch.Generator(device=d).manual_seed(18)
    kc = torch.randn(nb, bs, hkv, 128, generator=dg, device=d, dtype=torch.bfloat16)
    vc = torch.randn(nb, bs, hkv, 128, generator=dg, device=d, dtype=torch.bfloat16)
    q = randn_bf16((B, hq, 128), g).to(d)
    ctx_d, bt_d = ctx.to(d), bt.to(d)
    out = _decode(q, kc, vc, ctx_d, bt_d)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    _device_oracle_check(q, kc, vc, bt_d, ctx_d, out)
    del kc, vc
    torch.cuda.empty_cache()


def test_decode_golden(cuda_device):
    f = load("decode_small")
    d = cuda_device
    out = _decode(bf16(f["q"]).to(d), bf16(f["k_cache"]).to(d), bf16(f["v_cache"]).to(d),
                  torch.from_numpy(f["context_lens"]).to(d), torch.from_numpy(f["block_tables"]).to(d),
                  scale=float(f["scale"]))
    torch.cuda.synchronize()
    torch.testing.assert_close(out.cpu().double(), torch.from_numpy(f["out"]), **TOL)
    # one-token row: exactly the V row
    assert np.array_equal(out[0].cpu().float().numpy(), f["out"][0].astype(np.float32))


def test_decode_one_long_sequence_spans_the_grid(cuda_device):
    """A single 32k-token context (plus a 1-token one): the stream-K split cuts it into
    many ranges across the whole grid and the merge combines them."""
    g = gen(31)
    ctx = torch.tensor([32768, 1], dtype=torch.int32)
    nb = 128 + 1 + 3
    _, kc, vc = interleaved_pool(nb, 256, 8, 128, g)
    bt = random_block_tables([32768, 1], 256, nb, g)
    q = randn_bf16((2, 16, 128), g)
    _check(cuda_device, q, kc, vc, bt, ctx)


def test_decode_batch_above_one_launch(cuda_device):
    """More sequences than one launch's prefix-sum table holds (4096): the host splits
    the batch into consecutive launches that share the workspace."""
    B = 4100
    q, kc, vc, bt, ctx = _case(32, B=B, hq=4, hkv=2, bs=64, lo=0, hi=70)
    _check(cuda_device, q, kc, vc, bt, ctx)


def test_decode_block_size_512_and_strided_query(cuda_device):
    """512-token pages, and q given as a strided view of the fused qkv rows (row stride
    (Hq + 2 Hkv) * D, as the model produces it)."""
    hq, hkv, B = 8, 4, 6
    q0, kc, vc, bt, ctx = _case(33, B=B, hq=hq, hkv=hkv, bs=512, lo=1, hi=3000)
    g = gen(34)
    qkv = randn_bf16((B, (hq + 2 * hkv) * 128), g)
    qkv[:, :hq * 128] = q0.reshape(B, -1)
    qv = qkv[:, :hq * 128].view(B, hq, 128)
    assert qv.stride(0) == (hq + 2 * hkv) * 128
    d = cuda_device
    out = _decode(qkv.to(d)[:, :hq * 128].view(B, hq, 128), kc.to(d), vc.to(d), ctx.to(d), bt.to(d))
    torch.cuda.synchronize()
    torch.testing.assert_close(out.cpu().float(), ref.paged_decode(q0, kc, vc, bt, ctx, SCALE), **TOL)


def test_decode_back_to_back_shapes_share_the_workspace(cuda_device):
    """Back-to-back calls of different shapes on the one per-device workspace (each
    later call laying its partial states over an earlier call's) all match the oracle.
    The cases cover every GQA ratio and sequences cut into many parts."""
    d = cuda_device
    cases = [(40, 8, 1, 64, 4000, 9000), (3, 64, 8, 256, 20000, 30000), (64, 16, 8, 256, 1, 2048),
             (7, 8, 2, 128, 900, 5000), (5, 16, 4, 64, 3000, 7000), (24, 40, 8, 256, 1, 4000)]
    for i, (B, hq, hkv, bs, lo, hi) in enumerate(cases):
        q, kc, vc, bt, ctx = _case(40 + i, B=B, hq=hq, hkv=hkv, bs=bs, lo=lo, hi=hi)
        _check(d, q, kc, vc, bt, ctx)


def test_decode_relocated_pages_are_bitwise_identical(cuda_device):
    """Moving every page to another physical block and renumbering the tables to match
    changes no bit of the output: the split and the arithmetic depend on the logical
    tokens only."""
    q, kc, vc, bt, ctx = _case(50, B=24, hq=16, hkv=8, bs=256, lo=1, hi=3000, layout="interleaved")
    k2, v2, bt2 = relocate_pages(kc, vc, bt, gen(51))
    d = cuda_device
    a = _decode(q.to(d), kc.to(d), vc.to(d), ctx.to(d), bt.to(d)).cpu()
    b = _decode(q.to(d), k2.to(d), v2.to(d), ctx.to(d), bt2.to(d)).cpu()
    assert bits_equal(a, b)
    torch.testing.assert_close(a.float(), ref.paged_decode(q, kc, vc, bt, ctx, SCALE), **TOL)
