"""CPU checks of the C ABI: libkvpath.so loads, exports exactly what include/kvpath.h
declares, and rejects bad arguments on the host before launching anything (these calls
make no HIP API call, so they run without a GPU)."""

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from kavor_amd import _lib

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "kvpath.h"


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(kvp_\w+)\s*\(", text)))


def test_header_matches_binding_table():
    assert declared_functions() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    for name in declared_functions():
        assert hasattr(lib, name), name
    nm = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True)
    exported = set(re.findall(r"\bT (kvp_\w+)$", nm.stdout, flags=re.M))
    assert exported == set(declared_functions())


def test_version_string():
    assert _lib.version().startswith("kvpath ")


def _append(**over):
    args = dict(key=16, kts=1024, khs=128, value=16, vts=4096, vhs=128, kc=16, vc=16,
                bstr=524288, sstr=1024, hstr=128, nslots=1 << 17, slots=16, n=4,
                hkv=8, d=128, bs=256, stream=None)
    args.update(over)
    return _lib.lib().kvp_append_bf16(*args.values())


def test_append_rejects_bad_arguments_on_host():
    lib = _lib.lib()
    assert _append(n=0) == _lib.KVP_OK                       # nothing to do
    assert _append(d=96) == _lib.KVP_EUNSUPPORTED
    assert b"head_dim=96" in lib.kvp_last_error()
    assert _append(key=8) == _lib.KVP_EINVAL                 # misaligned pointer
    assert _append(vts=4100) == _lib.KVP_EINVAL              # stride not a multiple of 8
    assert _append(slots=0) == _lib.KVP_EINVAL               # null slot mapping
    assert _append(n=-1) == _lib.KVP_EINVAL


def _decode(**over):
    args = dict(q=16, qs=2048, qh=128, kc=16, vc=16, bstr=524288, sstr=1024, hstr=128, nblk=64,
                bt=16, bts=16, ctx=16, b=4, hq=16, hkv=8, d=128, bs=256, maxb=16, scale=0.088,
                out=16, os=2048, oh=128, ws=256, wsb=1 << 30, stream=None)
    args.update(over)
    return _lib.lib().kvp_paged_decode_bf16(*args.values())


def test_decode_rejects_bad_arguments_on_host():
    assert _decode(b=0) == _lib.KVP_OK
    assert _decode(d=64) == _lib.KVP_EUNSUPPORTED
    assert _decode(hq=12) == _lib.KVP_EINVAL                 # 12 q heads over 8 kv heads
    assert _decode(hq=24) == _lib.KVP_EUNSUPPORTED           # GQA ratio 3
    assert _decode(bs=100) == _lib.KVP_EINVAL                # not a multiple of 64
    assert _decode(bts=8) == _lib.KVP_EINVAL                 # table stride < width
    assert _decode(wsb=100) == _lib.KVP_EWORKSPACE           # smaller than the header
    assert _decode(ws=32) == _lib.KVP_EINVAL                 # not 256-byte aligned
    assert b"workspace" in _lib.lib().kvp_last_error()


def test_noalloc_decode_rejects_bad_arguments_on_host():
    lib = _lib.lib()
    args = dict(q=16, qs=2048, qh=128, kc=16, vc=16, bstr=524288, sstr=1024, hstr=128, nblk=64,
                bt=16, bts=16, ctx=16, b=4, hq=16, hkv=8, d=128, bs=256, maxb=16, scale=0.088,
                out=16, os=2048, oh=128, stream=None)

    def call(**over):
        return lib.kvp_paged_decode_bf16_noalloc(*dict(args, **over).values())

    assert call(b=0) == _lib.KVP_OK
    assert call(d=64) == _lib.KVP_EUNSUPPORTED
    assert call(hq=24) == _lib.KVP_EUNSUPPORTED
    assert call(bs=100) == _lib.KVP_EINVAL
    assert call(out=None) == _lib.KVP_EINVAL
    assert b"kvp_paged_decode_bf16_noalloc" in lib.kvp_last_error()


def test_sample_rejects_bad_arguments_on_host():
    lib = _lib.lib()
    args = dict(logits=16, rs=151936, rows=4, vocab=151936, temps=16, seed=16, out=16, ws=None, wsb=0,
                stream=None)

    def call(**over):
        return lib.kvp_sample_bf16(*dict(args, **over).values())

    assert call(rows=0) == _lib.KVP_OK
    assert call(temps=None) == _lib.KVP_EINVAL
    assert call(seed=None) == _lib.KVP_EINVAL
    assert call(seed=18) == _lib.KVP_EINVAL                  # not 4-byte aligned
    assert call(rs=151937) == _lib.KVP_EINVAL                # stride not a multiple of 8
    assert call(logits=8) == _lib.KVP_EINVAL                 # logits not 16-byte aligned
    assert call(vocab=0) == _lib.KVP_EINVAL
    assert call(ws=12) == _lib.KVP_EINVAL                    # workspace not 8-byte aligned


def test_fused_decode_rejects_bad_arguments_on_host():
    lib = _lib.lib()
    args = dict(qkv=16, qkvs=4096, cs=16, maxpos=40960, qw=16, kw=16, eps=1e-6, kc=16, vc=16,
                bstr=524288, sstr=1024, hstr=128, nblk=64, slots=16, bt=16, bts=16, ctx=16, b=4, hq=16, hkv=8,
                d=128, bs=256, maxb=16, scale=0.088, out=16, os=2048, oh=128, ws=256, wsb=1 << 30, stream=None)

    def call(**over):
        return lib.kvp_paged_decode_fused_bf16(*dict(args, **over).values())

    assert call(b=0) == _lib.KVP_OK
    assert call(cs=None) == _lib.KVP_EINVAL
    assert call(slots=None) == _lib.KVP_EINVAL
    assert call(maxpos=0) == _lib.KVP_EINVAL
    assert call(maxpos=1 << 23) == _lib.KVP_EINVAL           # table beyond 32-bit byte offsets
    assert call(qkvs=3000) == _lib.KVP_EINVAL                # row shorter than (hq + 2 hkv) * 128
    assert call(wsb=100) == _lib.KVP_EWORKSPACE
    assert b"kvp_paged_decode_fused_bf16" in lib.kvp_last_error()


def test_decode_workspace_size_formula():
    # 256-byte-aligned header (16 ints + a 4097-entry prefix table), then one state of 130
    # floats per query head for each of (ranges + sequences) slots; a launch has at most
    # min(1024, ceil(sequences * width * block_size / 128)) ranges
    header = ((16 + 4097) * 4 + 255) // 256 * 256
    state = 130 * 4
    size = _lib.lib().kvp_decode_workspace_bytes
    assert size(512, 16, 128, 16, 256) == header + (1024 + 512) * 16 * state
    assert size(9000, 16, 128, 16, 256) == header + (1024 + 4096) * 16 * state
    assert size(2, 16, 128, 1, 64) == header + (1 + 2) * 16 * state
    assert size(6, 32, 128, 2, 256) == header + (24 + 6) * 32 * state
    assert size(0, 16, 128, 16, 256) == 0
    assert size(8, 16, 64, 16, 256) == 0


def _prefill(**over):
    args = dict(q=16, qts=2048, qhs=128, k=16, kbs=0, kts=1024, khs=128, v=16, vbs=0, vts=4096,
                vhs=128, bt=None, bts=0, nblk=0, bs=0, maxb=0, cuq=16, cuk=16, nseq=2, maxq=100,
                hq=16, hkv=8, d=128, scale=0.088, causal=1, out=16, ots=2048, ohs=128, ws=256, wsb=1 << 30,
                stream=None)
    args.update(over)
    return _lib.lib().kvp_varlen_prefill_bf16(*args.values())


def test_prefill_rejects_bad_arguments_on_host():
    assert _prefill(nseq=0) == _lib.KVP_OK
    assert _prefill(d=256) == _lib.KVP_EUNSUPPORTED
    assert _prefill(bt=16, bs=32, maxb=4, bts=4, nblk=8) == _lib.KVP_EINVAL  # paged, bs % 64
    assert _prefill(kts=1020) == _lib.KVP_EINVAL
    assert _prefill(vts=1 << 24) == _lib.KVP_EINVAL              # 64 rows beyond 32-bit offsets
    assert b"token strides" in _lib.lib().kvp_last_error()
    assert _prefill(cuq=None) == _lib.KVP_EINVAL
    assert _prefill(wsb=100) == _lib.KVP_EWORKSPACE              # smaller than the work list
    assert b"workspace" in _lib.lib().kvp_last_error()
    assert _prefill(ws=None) == _lib.KVP_EWORKSPACE
    assert _prefill(ws=64) == _lib.KVP_EINVAL                    # not 256-byte aligned
    assert _prefill(out=24) == _lib.KVP_EINVAL                   # out rows are stored 16 bytes at a time
    assert _prefill(ots=2044) == _lib.KVP_EINVAL
    assert b"out" in _lib.lib().kvp_last_error()


def test_prefill_workspace_size_formula():
    # 2 KiB (claim counters, unit count) plus 32 bytes per (sequence, pair of query tiles);
    # a tile holds 128 / G query tokens; at most 2048 sequences per launch
    size = _lib.lib().kvp_prefill_workspace_bytes
    assert size(32, 1024, 16, 8) == 2048 + 32 * 32 * 8          # G = 2: 16 tiles, 8 pairs
    assert size(256, 4096, 16, 8) == 2048 + 32 * 256 * 32
    assert size(3, 100, 40, 8) == 2048 + 32 * 3 * 2             # G = 5: 25-token tiles, 4 tiles
    assert size(5000, 1, 8, 1) == 2048 + 32 * 2048 * 1           # G = 8, capped at one launch
    assert size(4, 0, 16, 8) == 2048
    assert size(4, 100, 24, 8) == 0                              # GQA ratio 3
    assert size(4, 100, 12, 8) == 0


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "libkvpath.so")
    with pytest.raises(RuntimeError, match="missing"):
        _lib.lib()
