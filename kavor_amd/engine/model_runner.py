"""Runs the model over the paged KV cache on one GPU: pool sizing, per-step metadata,
hipGraph decode.

Counterpart of kavor/engine/model_runner.py for one GPU (tensor_parallel_size=1, so
the shared-memory control plane of :85-106 has nothing to do):

- allocate_kv_cache (:329-383): a temporary pool serves a worst-case prefill and a
  full-batch decode whose activation peaks are measured; the page pool then takes
  total * gpu_memory_utilization - used - reserve (cache_pool.py:292-307);
- warmup_model / _profile_decode (:128-169): synthetic worst-case prefill (each
  sequence on its own consecutive blocks) and decode (all slots 0, context length 1);
- capture_cudagraph (:264-327): one hipGraph per batch size in
  [1, 2, 4, 8] + range(16, max_bs + 1, 16) (+ max_bs), sharing one memory pool,
  captured with all-zero metadata; as at tensor_parallel_size 1 there (:280-310), the
  LM head and the sampler are inside the graph, which leaves the tokens in a
  persistent sampled_tokens buffer (the rows' temperatures travel with the decode
  metadata, the sampler's seed is a device buffer the graph advances); the paged-decode workspace is reserved before
  capture;
- run / run_model (:213-262): prefill runs eagerly, decode replays the smallest graph
  that holds the batch, padding rows carry slot -1 and context length 0.

Per-step metadata travels in one host-to-device copy (kavor_amd.engine.metadata).  With
the fused layers the prefill always carries block tables, because the model appends
k / v before attention and attention reads the pages; with the drop-in caller order it
carries them only when some sequence has cached tokens (:432-433).  A decode batch that a graph holds reads its tokens from the
graph's sampled_tokens, at any temperature.
"""

from __future__ import annotations

import math
from time import perf_counter

import torch

from kavor_amd._lib import lib
from kavor_amd.config import Config
from kavor_amd.engine.cache_pool import CachePool
from kavor_amd.engine.metadata import DecodeStaging, prepare_prefill
from kavor_amd.engine.qwen3 import Qwen3ForCausalLM, load_checkpoint_tensors
from kavor_amd.engine.sampler import Sampler
from kavor_amd.engine.sequence import Sequence
from kavor_amd.layers.attention import reserve_decode_workspace
from kavor_amd.layers.fused import argmax_workspace
from kavor_amd.utils.context import reset_context, set_context

MAX_GRAPH_BATCH = 512


def graph_batch_sizes(max_bs: int) -> list[int]:
    sizes = [b for b in (1, 2, 4, 8) if b <= max_bs] + list(range(16, max_bs + 1, 16))
    if sizes[-1] != max_bs:
        sizes.append(max_bs)
    return sizes


class ModelRunner:

    def __init__(self, config: Config):
        if not torch.cuda.is_available():
            raise RuntimeError("ModelRunner needs a GPU (MI355X / gfx950)")
        lib()  # the paged KV path has no other implementation: fail here if it is missing
        self.config = config
        self.spec = config.spec
        self.block_size = config.kvcache_block_size
        self.device = torch.device("cuda", torch.cuda.current_device())
        self.max_blocks = math.ceil(config.max_model_len / self.block_size)
        self.timings = {"load": 0.0, "pool": 0.0, "capture": 0.0}

        t0 = perf_counter()
        self.model = Qwen3ForCausalLM(self.spec, self.device, caller=config.attention_caller,
                                      fused_decode=config.fused_decode)
        if config.checkpoint is not None:
            tensors = load_checkpoint_tensors(config.checkpoint)
            self.model.load_hf_state({k: v.to(self.device) for k, v in tensors.items()})
            del tensors
        else:
            self.model.init_random(config.seed)
        self.sampler = Sampler(self.device)
        self.pool = CachePool(self.model, self.spec.num_key_value_heads, self.spec.head_dim,
                              self.block_size)
        torch.cuda.synchronize()
        self.timings["load"] = perf_counter() - t0

        t0 = perf_counter()
        self.allocate_kv_cache()
        self.timings["pool"] = perf_counter() - t0
        self.staging = DecodeStaging(config.max_num_seqs, self.max_blocks, self.device)
        self.graphs: dict[int, torch.cuda.CUDAGraph] = {}
        self.graph_bs: list[int] = []
        if not config.enforce_eager:
            t0 = perf_counter()
            self.capture_graphs()
            self.timings["capture"] = perf_counter() - t0

    # ------------------------------------------------------------------ synthetic passes

    def _prefill_shape(self) -> tuple[int, int]:
        seq_len = min(self.config.max_num_batched_tokens, self.config.max_model_len)
        num_seqs = max(1, min(self.config.max_num_batched_tokens // seq_len, self.config.max_num_seqs))
        return seq_len, num_seqs

    @torch.inference_mode()
    def warmup_model(self) -> None:
        """Worst-case prefill: sequence i owns blocks [i*n, (i+1)*n) of the bound pool."""
        seq_len, num_seqs = self._prefill_shape()
        nb = math.ceil(seq_len / self.block_size)
        total = seq_len * num_seqs
        dev = self.device
        ids = torch.zeros(total, dtype=torch.int32, device=dev)
        p = torch.arange(seq_len, dtype=torch.int32, device=dev)
        pos = p.repeat(num_seqs)
        tables = torch.arange(num_seqs * nb, dtype=torch.int32, device=dev).view(num_seqs, nb)
        slots = (tables[:, p // self.block_size] * self.block_size + p % self.block_size).reshape(-1)
        cu = torch.arange(0, total + 1, seq_len, dtype=torch.int32, device=dev)
        set_context(True, cu, cu, seq_len, seq_len, slots.contiguous(), None,
                    tables if self.model.prefill_reads_pages else None)
        try:
            logits = self.model.compute_logits(self.model(ids, pos))
            self.sampler(logits, None, True)
        finally:
            reset_context()

    @torch.inference_mode()
    def profile_decode(self, bs: int) -> None:
        dev = self.device
        set_context(False, slot_mapping=torch.zeros(bs, dtype=torch.int32, device=dev),
                    context_lens=torch.ones(bs, dtype=torch.int32, device=dev),
                    block_tables=torch.zeros(bs, 1, dtype=torch.int32, device=dev))
        try:
            zeros = torch.zeros(bs, dtype=torch.int32, device=dev)
            logits = self.model.compute_logits(self.model(zeros, zeros))
            self.sampler(logits, torch.ones(bs, dtype=torch.float32, device=dev), False)
        finally:
            reset_context()

    def _peak(self, fn) -> int:
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        torch.cuda.reset_peak_memory_stats()
        base = torch.cuda.memory_allocated()
        fn()
        torch.cuda.synchronize()
        return torch.cuda.max_memory_allocated() - base

    # ------------------------------------------------------------------ page pool

    def allocate_kv_cache(self) -> None:
        cfg = self.config
        seq_len, num_seqs = self._prefill_shape()
        probe_blocks = num_seqs * math.ceil(seq_len / self.block_size) + 2
        decode_bs = min(cfg.max_num_seqs, MAX_GRAPH_BATCH)
        reserve_decode_workspace(decode_bs, self.spec.num_attention_heads, self.spec.head_dim,
                                 self.max_blocks, self.block_size, self.device)
        if cfg.num_kvcache_blocks > 0:
            num_blocks = cfg.num_kvcache_blocks
            self.pool.allocate(max(num_blocks, probe_blocks), self.device)
            self.warmup_model()
            if num_blocks < probe_blocks:
                self.pool.allocate(num_blocks, self.device)
        else:
            self.pool.allocate(probe_blocks, self.device)
            prefill_peak = self._peak(self.warmup_model)
            decode_peak = self._peak(lambda: self.profile_decode(decode_bs))
            graph_pool = 0 if cfg.enforce_eager else decode_peak
            reserve = graph_pool + max(prefill_peak, decode_peak)
            self.pool.release()
            torch.cuda.synchronize()
            torch.cuda.empty_cache()
            free, total = torch.cuda.mem_get_info()
            budget = int(total * cfg.gpu_memory_utilization) - (total - free) - reserve
            num_blocks = self.pool.blocks_for_budget(budget)
            if num_blocks < 1:
                raise RuntimeError(
                    f"no room for the page pool: budget {budget / 2**30:.2f} GiB after "
                    f"{reserve / 2**30:.2f} GiB of activations; lower max_num_seqs / "
                    "max_num_batched_tokens or raise gpu_memory_utilization")
            self.pool.allocate(num_blocks, self.device)
        cfg.num_kvcache_blocks = num_blocks
        if num_blocks < cfg.max_num_seqs:
            cfg.max_num_seqs = num_blocks  # each running sequence holds at least one page

    # ------------------------------------------------------------------ graphs

    @torch.inference_mode()
    def capture_graphs(self) -> None:
        spec = self.spec
        max_bs = min(self.config.max_num_seqs, MAX_GRAPH_BATCH)
        reserve_decode_workspace(max_bs, spec.num_attention_heads, spec.head_dim,
                                 self.max_blocks, self.block_size, self.device)
        self.logits_buf = torch.empty(max_bs, spec.vocab_size, dtype=torch.bfloat16, device=self.device)
        self.sampled_buf = torch.zeros(max_bs, dtype=torch.int64, device=self.device)
        argmax_workspace(self.device)
        self.graph_bs = graph_batch_sizes(max_bs)
        pool = None
        # all-zero metadata: context length 0 rows and slot 0 (model_runner.py:272-274)
        self.staging.dev.zero_()
        for bs in reversed(self.graph_bs):
            m = self.staging.views(bs)
            set_context(False, slot_mapping=m.slot_mapping, context_lens=m.context_lens,
                        block_tables=m.block_tables)
            try:
                out, tok = self.logits_buf[:bs], self.sampled_buf[:bs]
                self.sampler(self.model.compute_logits(self.model(m.input_ids, m.positions), out=out),
                             m.temperatures, False, out=tok)
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, pool=pool):
                    self.sampler(self.model.compute_logits(self.model(m.input_ids, m.positions), out=out),
                                 m.temperatures, False, out=tok)
            finally:
                reset_context()
            if pool is None:
                pool = graph.pool()
            self.graphs[bs] = graph
            torch.cuda.synchronize()
        self.graph_pool = pool

    # ------------------------------------------------------------------ steps

    @torch.inference_mode()
    def run(self, seqs: list[Sequence], is_prefill: bool) -> list[int]:
        temps = [s.temperature for s in seqs]
        all_greedy = all(t == 0.0 for t in temps)
        try:
            if is_prefill:
                m = prepare_prefill(seqs, self.block_size, self.device,
                                    always_tables=self.model.prefill_reads_pages)
                set_context(True, m.cu_seqlens_q, m.cu_seqlens_k, m.max_seqlen_q, m.max_seqlen_k,
                            m.slot_mapping, None, m.block_tables)
                logits = self.model.compute_logits(self.model(m.input_ids, m.positions))
            else:
                logits, sampled, t = self._decode(seqs)
                if sampled is not None:
                    return sampled.tolist()  # the graph's LM head + sampler
                return self.sampler(logits, t, all_greedy).tolist()
            t = None if all_greedy else torch.tensor(temps, dtype=torch.float32).to(self.device, non_blocking=True)
            return self.sampler(logits, t, all_greedy).tolist()
        finally:
            reset_context()

    def _decode(self, seqs: list[Sequence]) -> tuple[torch.Tensor, torch.Tensor | None, torch.Tensor]:
        """Logits of a decode step, the sampled tokens when a graph produced them, and the
        rows' temperatures on the device."""
        n = len(seqs)
        if self.graphs and n <= self.graph_bs[-1]:
            bs = next(b for b in self.graph_bs if b >= n)
            self.staging.fill(seqs, self.block_size, bs)
            self.graphs[bs].replay()
            return self.logits_buf[:n], self.sampled_buf[:n], self.staging.views(n).temperatures
        self.staging.fill(seqs, self.block_size, n)
        m = self.staging.views(n)
        set_context(False, slot_mapping=m.slot_mapping, context_lens=m.context_lens,
                    block_tables=m.block_tables)
        return self.model.compute_logits(self.model(m.input_ids, m.positions)), None, m.temperatures

    def exit(self) -> None:
        self.graphs.clear()
        self.pool.release()
        torch.cuda.synchronize()
