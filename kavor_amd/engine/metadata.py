"""Per-step metadata of the paged KV path, built on the host and shipped in one copy.

Same values as ModelRunner.prepare_prefill / prepare_decode / prepare_block_tables
(kavor/engine/model_runner.py:385-473):

prefill, for the scheduled tokens [num_cached, num_cached + num_scheduled) of each
sequence:  input_ids, positions, slot_mapping[t] = block_table[pos // bs] * bs + pos % bs,
cu_seqlens_q / cu_seqlens_k (k counts the cached prefix too), max_seqlen_q/k, and the
block tables (rows right-padded with -1) only when some sequence has cached tokens,
i.e. sum(klen) > sum(qlen) (model_runner.py:432-433);

decode, one token per sequence:  input_ids = last token, position = len - 1,
slot = block_table[-1] * bs + last_block_num_tokens - 1, context_len = len (the token
being appended counts), block tables right-padded with -1.

Instead of one pinned tensor and one host-to-device copy per field, every field is
packed into a single int32 buffer that moves in one copy; the device tensors the model
and the kernels read are views into it.  Decode uses a fixed layout with `rows` rows
(the captured graph size) so graph replays read the same addresses every step:
padding rows get slot -1 and context length 0, which the append skips and the decode
writes as zeros, and block-table columns past a sequence's length are never read.
"""

from __future__ import annotations

from dataclasses import dataclass
from itertools import chain

import numpy as np
import torch

from kavor_amd.engine.sequence import Sequence


@dataclass
class PrefillMeta:
    input_ids: torch.Tensor
    positions: torch.Tensor
    slot_mapping: torch.Tensor
    cu_seqlens_q: torch.Tensor
    cu_seqlens_k: torch.Tensor
    max_seqlen_q: int
    max_seqlen_k: int
    block_tables: torch.Tensor | None


@dataclass
class DecodeMeta:
    input_ids: torch.Tensor
    positions: torch.Tensor
    slot_mapping: torch.Tensor
    context_lens: torch.Tensor
    block_tables: torch.Tensor
    temperatures: torch.Tensor  # fp32, 0 for greedy rows and padding


def _pinned_int32(n: int, pin: bool) -> torch.Tensor:
    return torch.empty(n, dtype=torch.int32, pin_memory=pin)


def prefill_arrays(seqs: list[Sequence], block_size: int, always_tables: bool = False):
    """Host arrays of a prefill step (numpy int32); see the module docstring.  With
    always_tables the block tables are produced even without cached tokens (attention
    that reads the pages for every prefill needs them)."""
    n = len(seqs)
    qlens = np.fromiter((s.num_scheduled_tokens for s in seqs), dtype=np.int64, count=n)
    starts = np.fromiter((s.num_cached_tokens for s in seqs), dtype=np.int64, count=n)
    if (qlens <= 0).any():
        raise ValueError("every prefill sequence needs at least one scheduled token")
    klens = starts + qlens
    T = int(qlens.sum())
    ids = np.empty(T, dtype=np.int32)
    pos = np.empty(T, dtype=np.int32)
    slots = np.empty(T, dtype=np.int32)
    o = 0
    for s, start, ql in zip(seqs, starts.tolist(), qlens.tolist()):
        end = start + ql
        if len(s.block_table) * block_size < end:
            raise ValueError(f"sequence {s.seq_id} has {len(s.block_table)} blocks for {end} tokens")
        p = np.arange(start, end, dtype=np.int64)
        table = np.asarray(s.block_table, dtype=np.int64)
        ids[o:o + ql] = s.token_ids[start:end]
        pos[o:o + ql] = p
        slots[o:o + ql] = table[p // block_size] * block_size + p % block_size
        o += ql
    cu_q = np.zeros(n + 1, dtype=np.int32)
    cu_k = np.zeros(n + 1, dtype=np.int32)
    cu_q[1:] = np.cumsum(qlens)
    cu_k[1:] = np.cumsum(klens)
    tables = None
    if always_tables or int(klens.sum()) > T:
        width = max(len(s.block_table) for s in seqs)
        tables = np.full((n, width), -1, dtype=np.int32)
        for i, s in enumerate(seqs):
            tables[i, :len(s.block_table)] = s.block_table
    return dict(input_ids=ids, positions=pos, slot_mapping=slots, cu_seqlens_q=cu_q,
                cu_seqlens_k=cu_k, max_seqlen_q=int(qlens.max()), max_seqlen_k=int(klens.max()),
                block_tables=tables)


def prepare_prefill(seqs: list[Sequence], block_size: int, device, pin: bool = True,
                    always_tables: bool = False) -> PrefillMeta:
    a = prefill_arrays(seqs, block_size, always_tables)
    parts = [a["input_ids"], a["positions"], a["slot_mapping"], a["cu_seqlens_q"], a["cu_seqlens_k"]]
    if a["block_tables"] is not None:
        parts.append(a["block_tables"].reshape(-1))
    sizes = [p.size for p in parts]
    host = _pinned_int32(sum(sizes), pin)
    np.concatenate(parts, out=host.numpy())
    dev = host.to(device, non_blocking=True)
    views = list(torch.split(dev, sizes))
    tables = views[5].view(len(seqs), -1) if a["block_tables"] is not None else None
    return PrefillMeta(views[0], views[1], views[2], views[3], views[4],
                       a["max_seqlen_q"], a["max_seqlen_k"], tables)


class DecodeStaging:
    """Fixed-layout decode metadata: [ids | positions | slots | context_lens |
    temperatures (fp32 bits) | tables] with `rows` rows and `width` block-table columns,
    in one pinned host buffer and one device buffer.  `views(bs)` returns the device
    views of the first bs rows."""

    def __init__(self, rows: int, width: int, device, pin: bool = True):
        self.rows, self.width = rows, width
        self.host = _pinned_int32(rows * (5 + width), pin)
        self.h = self.host.numpy()
        self.dev = torch.zeros(rows * (5 + width), dtype=torch.int32, device=device)
        self.h[:] = 0
        self._hf = [self.h[i * rows:(i + 1) * rows] for i in range(4)]
        self._htemp = self.h[4 * rows:5 * rows].view(np.float32)
        self._htab = self.h[5 * rows:].reshape(rows, width)
        self._df = [self.dev[i * rows:(i + 1) * rows] for i in range(4)]
        self._dtemp = self.dev[4 * rows:5 * rows].view(torch.float32)
        self._dtab = self.dev[5 * rows:].view(rows, width)

    def views(self, bs: int) -> DecodeMeta:
        ids, pos, slots, ctx = (t[:bs] for t in self._df)
        return DecodeMeta(ids, pos, slots, ctx, self._dtab[:bs], self._dtemp[:bs])

    def fill(self, seqs: list[Sequence], block_size: int, bs: int) -> None:
        """Writes the host rows for `seqs`, pads rows len(seqs)..bs-1, and copies the
        buffer to the device (non-blocking, on the current stream).  The caller must
        not refill before that copy has completed (the engine synchronises every step).

        One pass over the sequences per field, then array operations: the ragged block
        tables are scattered with one boolean-mask assignment (row i gets its table and
        a -1 after it when it is narrower than the buffer; later columns keep stale
        entries, which the kernels never read)."""
        n = len(seqs)
        if n > bs or bs > self.rows:
            raise ValueError(f"{n} sequences do not fit {bs} rows (staging has {self.rows})")
        ids, pos, slots, ctx = self._hf
        L = np.fromiter((s.num_tokens for s in seqs), dtype=np.int64, count=n)
        nbs = np.fromiter((len(s.block_table) for s in seqs), dtype=np.int64, count=n)
        bad = (nbs * block_size < L) | (nbs > self.width)
        if bad.any():
            i = int(np.argmax(bad))
            raise ValueError(f"sequence {seqs[i].seq_id}: {int(nbs[i])} blocks for {int(L[i])} tokens "
                             f"(table width {self.width})")
        flat = np.fromiter(chain.from_iterable(s.block_table for s in seqs), dtype=np.int32,
                           count=int(nbs.sum()))
        starts = np.cumsum(nbs) - nbs
        self._htab[:n][np.arange(self.width)[None, :] < nbs[:, None]] = flat  # row-major = ragged order
        short = nbs < self.width
        self._htab[np.arange(n)[short], nbs[short]] = -1
        last = L - 1
        ids[:n] = np.fromiter((s.last_token for s in seqs), dtype=np.int64, count=n)
        pos[:n] = last
        ctx[:n] = L
        slots[:n] = flat[starts + last // block_size].astype(np.int64) * block_size + last % block_size
        ids[n:bs] = 0
        pos[n:bs] = 0
        slots[n:bs] = -1
        ctx[n:bs] = 0
        self._htemp[:n] = np.fromiter((s.temperature for s in seqs), dtype=np.float32, count=n)
        self._htemp[n:bs] = 0.0
        self.dev.copy_(self.host, non_blocking=True)


def decode_arrays(seqs: list[Sequence], block_size: int) -> dict:
    """Unpadded host arrays of a decode step (for tests and eager use)."""
    st = DecodeStaging(len(seqs), max(len(s.block_table) for s in seqs), "cpu", pin=False)
    st.fill(seqs, block_size, len(seqs))
    n, w = len(seqs), st.width
    ids, pos, slots, ctx = (f.copy() for f in st._hf)
    tab = st._htab.copy()
    for i, s in enumerate(seqs):
        tab[i, len(s.block_table):] = -1
    return dict(input_ids=ids[:n], positions=pos[:n], slot_mapping=slots[:n],
                context_lens=ctx[:n], block_tables=tab.reshape(n, w),
                temperatures=st._htemp[:n].copy())
