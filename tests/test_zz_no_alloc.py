"""The decode entry point that allocates nothing (kvp_paged_decode_bf16_noalloc), called
through the C ABI and compared with kvp_paged_decode_bf16 on a caller workspace.

Both run the same kernels with the same work split, so their outputs must agree bit for
bit; the first call is also checked against the fp32 oracle.  Two calls in a row, the
second with a smaller batch and another GQA ratio, show that what the first call left in
the shared static scratch does not leak into the second.  A batch whose partial states
do not fit the scratch is rejected before any launch.
"""

import ctypes

import pytest
import torch

from kavor_amd import _lib
from oracle import kvpath_oracle as ref
from tests.helpers import TOL, bits_equal, gen, interleaved_pool, random_block_tables, randn_bf16

pytestmark = pytest.mark.gpu
SCALE = 128 ** -0.5


def _inputs(dev, seed, B, hq, hkv, bs, lo, hi):
    g = gen(seed)
    ctx = torch.randint(lo, hi + 1, (B,), generator=g, dtype=torch.int32)
    nb = sum(-(-int(c) // bs) for c in ctx) + 2
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


def _run_both(dev, d):
    lib = _lib.lib()
    stream = torch.cuda.current_stream(dev).cuda_stream
    B, hq, D = d["q"].shape
    bs, width = d["kc"].shape[1], d["bt"].shape[1]
    out_static = torch.full((B, hq, D), float("nan"), dtype=torch.bfloat16, device=dev)
    out_ws = torch.empty_like(out_static)
    rc = lib.kvp_paged_decode_bf16_noalloc(*_args(d, out_static), stream)
    _lib.check("kvp_paged_decode_bf16_noalloc", rc)
    nbytes = lib.kvp_decode_workspace_bytes(B, hq, D, width, bs)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    rc = lib.kvp_paged_decode_bf16(*_args(d, out_ws), ws.data_ptr(), nbytes, stream)
    _lib.check("kvp_paged_decode_bf16", rc)
    torch.cuda.synchronize()
    return out_static.cpu(), out_ws.cpu()


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
