"""The decode entry point that allocates nothing (kvp_paged_decode_bf16_noalloc), called
through the C ABI and compared with kvp_paged_decode_bf16 on a caller workspace.

Both run the same kernels with the same work split, so their outputs must agree bit for
bit; each call is also checked against the fp32 oracle.  Two calls in a row, the
second with a smaller batch and another GQA ratio, show that what the first call left in
the shared static scratch does not leak into the second.  The GQA ratios 1, 5 and 8 run
too, including 4 kv heads or fewer (one head group per range, so a launch may use the
most ranges per head and the most scratch per sequence).  A graph that captured the call
is replayed with new metadata written into the same buffers, and each replay equals the
workspace entry point bit for bit.  A first call on a device inside a capture is refused
(the scratch address is looked up once, outside capture), and a batch whose partial
states do not fit the scratch is rejected before any launch.
"""

import ctypes
import os
import subprocess
import sys
import textwrap

import pytest
import torch

from kavor_amd import _lib
from oracle import kvpath_oracle as ref
from tests.helpers import TOL, bits_equal, gen, interleaved_pool, random_block_tables, randn_bf16

pytestmark = pytest.mark.gpu
SCALE = 128 ** -0.5


def _inputs(dev, seed, B, hq, hkv, bs, lo, hi, nb=None):
    g = gen(seed)
    ctx = torch.randint(lo, hi + 1, (B,), generator=g, dtype=torch.int32)
    nb = nb or sum(-(-int(c) // bs) for c in ctx) + 2
    _, kc, vc = interleaved_pool(nb, bs, hkv, 128, g)
    bt = random_block_tables([int(c) for c in ctx], bs, nb, g)
    q = randn_bf16((B, hq, 128), g)
    host = dict(q=q, kc=kc, vc=vc, bt=bt, ctx=ctx)
    return host, {k: v.to(dev) for k, v in host.items()}


def _args(d, out):
    q, kc, bt = d["q"], d["kc"], d["bt"]
    B, hq, D = q.shape
    nb, bs, hkv, _ = kc.shape
    return [q.data_ptr(), q.stride(0), q.stride(1),
            kc.data_ptr(), d["vc"].data_ptr(), kc.stride(0), kc.stride(1), kc.stride(2), nb,
            bt.data_ptr(), bt.stride(0), d["ctx"].data_ptr(), B, hq, hkv, D, bs, bt.shape[1],
            ctypes.c_float(SCALE), out.data_ptr(), out.stride(0), out.stride(1)]


def _workspace_call(dev, d):
    lib = _lib.lib()
    B, hq, D = d["q"].shape
    bs, width = d["kc"].shape[1], d["bt"].shape[1]
    out_ws = torch.empty((B, hq, D), dtype=torch.bfloat16, device=dev)
    nbytes = lib.kvp_decode_workspace_bytes(B, hq, D, width, bs)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    rc = lib.kvp_paged_decode_bf16(*_args(d, out_ws), ws.data_ptr(), nbytes,
                                   torch.cuda.current_stream(dev).cuda_stream)
    _lib.check("kvp_paged_decode_bf16", rc)
    torch.cuda.synchronize()
    return out_ws.cpu()


def _run_both(dev, d):
    lib = _lib.lib()
    B, hq, D = d["q"].shape
    out_static = torch.full((B, hq, D), float("nan"), dtype=torch.bfloat16, device=dev)
    rc = lib.kvp_paged_decode_bf16_noalloc(*_args(d, out_static), torch.cuda.current_stream(dev).cuda_stream)
    _lib.check("kvp_paged_decode_bf16_noalloc", rc)
    torch.cuda.synchronize()
    return out_static.cpu(), _workspace_call(dev, d)


def test_noalloc_decode_equals_workspace_decode_twice(cuda_device):
    # first call: the Qwen3-0.6B decode layer (G = 2, 256-token pages), long contexts
    host, d = _inputs(cuda_device, 31, B=64, hq=16, hkv=8, bs=256, lo=1, hi=2500)
    got, want = _run_both(cuda_device, d)
    assert bits_equal(got, want)
    sample = [0, 1, 17, 40, 63]
    oracle = ref.paged_decode(host["q"][sample], host["kc"], host["vc"], host["bt"][sample],
                              host["ctx"][sample], SCALE)
    torch.testing.assert_close(got[sample].float(), oracle, **TOL)

    # second call, smaller: 5 sequences, G = 4, 128-token pages
    host, d = _inputs(cuda_device, 32, B=5, hq=32, hkv=8, bs=128, lo=1, hi=900)
    got, want = _run_both(cuda_device, d)
    assert bits_equal(got, want)
    oracle = ref.paged_decode(host["q"], host["kc"], host["vc"], host["bt"], host["ctx"], SCALE)
    torch.testing.assert_close(got.float(), oracle, **TOL)


@pytest.mark.parametrize("B,hq,hkv,bs,lo,hi", [
    (24, 40, 8, 256, 1, 3000),    # G = 5 (Qwen3-14B heads)
    (20, 16, 2, 128, 1, 4000),    # G = 8, two kv heads: one head group per range
    (33, 4, 4, 64, 1, 5000),      # G = 1, four kv heads: one head group per range
    (3, 8, 1, 256, 5000, 9000),   # one kv head, a few long contexts: the most ranges per head
])
def test_noalloc_decode_gqa_shapes(cuda_device, B, hq, hkv, bs, lo, hi):
    host, d = _inputs(cuda_device, 33 + hq + hkv, B=B, hq=hq, hkv=hkv, bs=bs, lo=lo, hi=hi)
    got, want = _run_both(cuda_device, d)
    assert bits_equal(got, want)
    oracle = ref.paged_decode(host["q"], host["kc"], host["vc"], host["bt"], host["ctx"], SCALE)
    torch.testing.assert_close(got.float(), oracle, **TOL)


def test_noalloc_decode_graph_replay_with_new_metadata(cuda_device):
    """Captured once, replayed three times with new queries, contexts and tables written
    into the captured buffers; eager workspace calls on the host's copy of each input set
    run between the replays."""
    dev = cuda_device
    lib = _lib.lib()
    B, hq, hkv, bs, nb = 32, 16, 8, 256, 300
    host, d = _inputs(dev, 40, B=B, hq=hq, hkv=hkv, bs=bs, lo=1, hi=2048, nb=nb)
    width = 9  # every table below is padded to the captured width
    d["bt"] = torch.full((B, width), -1, dtype=torch.int32, device=dev)
    d["bt"][:, :host["bt"].shape[1]] = host["bt"].to(dev)
    out = torch.full((B, hq, 128), float("nan"), dtype=torch.bfloat16, device=dev)
    stream_args = lambda: torch.cuda.current_stream(dev).cuda_stream  # noqa: E731
    # one call outside capture sets the device's scratch address up
    _lib.check("kvp_paged_decode_bf16_noalloc", lib.kvp_paged_decode_bf16_noalloc(*_args(d, out), stream_args()))
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = lib.kvp_paged_decode_bf16_noalloc(*_args(d, out), stream_args())
    _lib.check("kvp_paged_decode_bf16_noalloc (captured)", rc)
    for rep in range(3):
        g = gen(50 + rep)
        ctx = torch.randint(1, width * bs + 1, (B,), generator=g, dtype=torch.int32)
        if rep == 1:
            ctx[::5] = 0  # padding rows, as the engine's graphs see them
        bt = random_block_tables([int(c) for c in ctx], bs, nb, g, width=width)
        if rep == 2:
            bt[bt < 0] = 7  # stale columns past each context must not be read
        q = randn_bf16((B, hq, 128), g)
        d["q"].copy_(q)
        d["ctx"].copy_(ctx)
        d["bt"].copy_(bt)
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = out.cpu()
        want = _workspace_call(dev, d)
        assert bits_equal(got, want), f"replay {rep}"
        live = [i for i in range(B) if int(ctx[i]) > 0]
        oracle = ref.paged_decode(q[live], host["kc"], host["vc"], bt[live], ctx[live], SCALE)
        torch.testing.assert_close(got[live].float(), oracle, **TOL)
        assert torch.all(got[[i for i in range(B) if int(ctx[i]) == 0]] == 0)


_FRESH_PROCESS_CAPTURE = textwrap.dedent("""
    import ctypes, sys, torch
    sys.path.insert(0, sys.argv[1])
    from kavor_amd import _lib
    lib = _lib.lib()
    dev = torch.device("cuda", 0)
    B, hq, hkv, bs = 4, 16, 8, 256
    q = torch.randn(B, hq, 128, device=dev).to(torch.bfloat16)
    kc = torch.randn(4, bs, hkv, 128, device=dev).to(torch.bfloat16)
    vc = torch.randn(4, bs, hkv, 128, device=dev).to(torch.bfloat16)
    bt = torch.arange(4, dtype=torch.int32, device=dev).view(B, 1)
    ctx = torch.full((B,), 100, dtype=torch.int32, device=dev)
    out = torch.zeros(B, hq, 128, dtype=torch.bfloat16, device=dev)
    args = [q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(), vc.data_ptr(), kc.stride(0),
            kc.stride(1), kc.stride(2), 4, bt.data_ptr(), bt.stride(0), ctx.data_ptr(), B, hq, hkv,
            128, bs, 1, ctypes.c_float(128 ** -0.5), out.data_ptr(), out.stride(0), out.stride(1)]
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc_captured = lib.kvp_paged_decode_bf16_noalloc(*args, torch.cuda.current_stream(dev).cuda_stream)
        msg = lib.kvp_last_error().decode()
    rc_eager = lib.kvp_paged_decode_bf16_noalloc(*args, torch.cuda.current_stream(dev).cuda_stream)
    torch.cuda.synchronize()
    print(rc_captured, rc_eager, bool(torch.isfinite(out.float()).all()), "|", msg, flush=True)
""")


def test_noalloc_first_call_inside_capture_is_refused(cuda_device):
    """In a fresh process, so that the scratch address is not yet cached: the captured
    first call returns KVP_EINVAL before any launch, and the eager call after it works."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    proc = subprocess.run([sys.executable, "-c", _FRESH_PROCESS_CAPTURE, root], capture_output=True,
                          text=True, timeout=110)
    assert proc.returncode == 0, proc.stderr[-2000:]
    head, msg = proc.stdout.strip().splitlines()[-1].split("|", 1)
    rc_captured, rc_eager, finite = head.split()
    assert int(rc_captured) == _lib.KVP_EINVAL
    assert "inside a graph capture" in msg
    assert int(rc_eager) == _lib.KVP_OK and finite == "True"


def test_noalloc_rejects_a_batch_beyond_the_scratch(cuda_device):
    """4096 sequences x 64 query heads need about 140 MB of partial states.  The buffers
    are sized for that batch (contexts 0, one page), so even a launch would stay in
    bounds; a launch would also overwrite the output with zeros."""
    lib = _lib.lib()
    dev = cuda_device
    B, hq, hkv, bs = 4096, 64, 8, 256
    q = torch.zeros(B, hq, 128, dtype=torch.bfloat16, device=dev)
    pool = torch.zeros(1, 2 * bs * hkv * 128, dtype=torch.bfloat16, device=dev)
    kc = pool[:, :bs * hkv * 128].view(1, bs, hkv, 128)
    vc = pool[:, bs * hkv * 128:].view(1, bs, hkv, 128)
    d = dict(q=q, kc=kc, vc=vc, bt=torch.zeros(B, 1, dtype=torch.int32, device=dev),
             ctx=torch.zeros(B, dtype=torch.int32, device=dev))
    out = torch.full((B, hq, 128), 3.0, dtype=torch.bfloat16, device=dev)
    rc = lib.kvp_paged_decode_bf16_noalloc(*_args(d, out), torch.cuda.current_stream(dev).cuda_stream)
    assert rc == _lib.KVP_EWORKSPACE
    assert b"static scratch" in lib.kvp_last_error()
    torch.cuda.synchronize()
    assert torch.all(out == 3.0)  # nothing was launched
