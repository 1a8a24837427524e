"""Writes tests/golden/philox_triton.npz (run from the repository root:
``python tests/golden/make_philox.py``): words and floats of Triton's own tl.randint /
tl.rand, computed by Triton's interpreter (TRITON_INTERPRET=1, on the CPU) with the
installed Triton, for int32 seeds read from memory and int32 offsets, as the reference's
sampler calls it (kavor/layers/sampler.py:34-38: seed loaded from an int32 buffer,
offsets i + r * V in int32 arithmetic).  The oracle's Philox restatement is checked
against these vectors.  No reference code is run: the kernel below is this file's own.
"""

from __future__ import annotations

import os
from pathlib import Path

os.environ["TRITON_INTERPRET"] = "1"

import numpy as np  # noqa: E402
import torch  # noqa: E402
import triton  # noqa: E402
import triton.language as tl  # noqa: E402

HERE = Path(__file__).resolve().parent
SEEDS = [0, 1, 2, 7, 123456789, 2**31 - 1, -1, -5, -2**31]
# offsets as int32: small, around the row boundaries of a 151936-wide vocabulary, near and
# past 2^31 (negative as int32, which the reference's int32 arithmetic produces)
OFFSETS = np.array(list(range(64)) + [151935, 151936, 151937, 255 * 151936 + 151935,
                                      2**31 - 2, 2**31 - 1, -2**31, -2**31 + 1, -2, -1],
                   dtype=np.int32)


@triton.jit
def _draw(seed_ptr, offs_ptr, words_ptr, floats_ptr, n, BLOCK: tl.constexpr):
    i = tl.arange(0, BLOCK)
    m = i < n
    seed = tl.load(seed_ptr)
    offs = tl.load(offs_ptr + i, mask=m, other=0)
    tl.store(words_ptr + i, tl.randint(seed, offs).to(tl.int32, bitcast=True), mask=m)
    tl.store(floats_ptr + i, tl.rand(seed, offs), mask=m)


def main() -> None:
    offs = torch.from_numpy(OFFSETS)
    n = offs.numel()
    words, floats = [], []
    for s in SEEDS:
        w = torch.zeros(n, dtype=torch.int32)
        f = torch.zeros(n, dtype=torch.float32)
        _draw[(1,)](torch.tensor([s], dtype=torch.int32), offs, w, f, n, BLOCK=triton.next_power_of_2(n))
        words.append(w.numpy().view(np.uint32).copy())
        floats.append(f.numpy().copy())
    np.savez_compressed(HERE / "philox_triton.npz", seeds=np.array(SEEDS, dtype=np.int64), offsets=OFFSETS,
                        words=np.stack(words), floats=np.stack(floats), triton_version=np.array(triton.__version__))
    print(f"wrote {HERE / 'philox_triton.npz'} ({len(SEEDS)} seeds x {n} offsets, triton {triton.__version__})")


if __name__ == "__main__":
    main()
