"""Offline generation API (kavor/engine/llm_engine.py:31-272, kavor/llm.py).

LLM(model, **config) builds the model runner (page pool, graphs) and the scheduler;
generate(prompts, sampling_params) submits every prompt, steps until all finish and
returns, in submission order, {"text", "token_ids"} per prompt, like the reference
(llm_engine.py:245-272).  Prompts are lists of token ids; text prompts and "text" in the
output need a tokenizer in the checkpoint directory (without one, "text" is None).

Every step's timing is kept in step_stats (prefill flag, scheduled tokens, step and
forward time), and finished requests in request_stats, as the reference's profile mode
records them (llm_engine.py:140-189), so decode throughput can be derived as
sum(decode tokens) / sum(decode step time) (benchs/decode_scaling.py:89-94).
"""

from __future__ import annotations

from dataclasses import fields
from pathlib import Path
from time import perf_counter

from kavor_amd.config import Config
from kavor_amd.engine.model_runner import ModelRunner
from kavor_amd.engine.scheduler import Scheduler
from kavor_amd.engine.sequence import Sequence
from kavor_amd.sampling_params import SamplingParams


def _load_tokenizer(path: str | None):
    if path is None or not (Path(path) / "tokenizer.json").exists():
        return None
    from transformers import AutoTokenizer

    return AutoTokenizer.from_pretrained(path, use_fast=True)


class LLMEngine:

    def __init__(self, model=None, **kwargs):
        names = {f.name for f in fields(Config) if f.init}
        unknown = set(kwargs) - names
        if unknown:
            raise TypeError(f"unknown engine options: {sorted(unknown)}")
        config = Config(model, **kwargs)
        self.config = config
        Sequence.block_size = config.kvcache_block_size
        self.model_runner = ModelRunner(config)   # sizes the pool, may lower max_num_seqs
        self.scheduler = Scheduler(config)
        self.tokenizer = _load_tokenizer(config.checkpoint)
        self.step_stats: list[dict] = []
        self.request_stats: list[dict] = []

    def exit(self) -> None:
        runner = getattr(self, "model_runner", None)
        if runner is not None:
            runner.exit()
            self.model_runner = None

    # ------------------------------------------------------------------ requests

    def add_request(self, prompt, sampling_params: SamplingParams, request_id: str | None = None) -> int:
        if isinstance(prompt, str):
            if self.tokenizer is None:
                raise ValueError("text prompts need a tokenizer in the checkpoint directory")
            prompt = self.tokenizer.encode(prompt)
        seq = Sequence(prompt, sampling_params)
        if seq.num_tokens + seq.max_tokens > self.config.max_model_len:
            raise ValueError(f"prompt ({seq.num_tokens}) + max_tokens ({seq.max_tokens}) exceeds "
                             f"max_model_len ({self.config.max_model_len})")
        seq.request_id = request_id
        self.scheduler.add(seq)
        return seq.seq_id

    def step(self) -> list[tuple[int, list[int]]]:
        start = perf_counter()
        seqs, is_prefill = self.scheduler.schedule()
        num_tokens = sum(s.num_scheduled_tokens for s in seqs)
        t_fwd = perf_counter()
        token_ids = self.model_runner.run(seqs, is_prefill)
        forward_time = perf_counter() - t_fwd
        now = perf_counter()
        if is_prefill:
            for s in seqs:
                if s.num_cached_tokens + s.num_scheduled_tokens == s.num_tokens:
                    s.stats.first_token_time = now
        self.scheduler.postprocess(seqs, token_ids, is_prefill)
        now = perf_counter()
        self.step_stats.append(dict(prefill=is_prefill, tokens=num_tokens, seqs=len(seqs),
                                    step_time=now - start, forward_time=forward_time))
        outputs = []
        for s in seqs:
            if s.is_finished:
                s.stats.finish_time = now
                self.request_stats.append(dict(
                    seq_id=s.seq_id, request_id=s.request_id,
                    num_prompt_tokens=s.num_prompt_tokens,
                    num_completion_tokens=s.num_completion_tokens,
                    arrival_time=s.stats.arrival_time,
                    prefill_start_time=s.stats.prefill_start_time,
                    first_token_time=s.stats.first_token_time, finish_time=now,
                    prefix_cache_hit_tokens=s.stats.prefix_cache_hit_tokens))
                outputs.append((s.seq_id, s.completion_token_ids))
        return outputs

    def is_finished(self) -> bool:
        return self.scheduler.is_finished()

    def generate(self, prompts, sampling_params, use_tqdm: bool = False) -> list[dict]:
        self.step_stats.clear()
        self.request_stats.clear()
        if not isinstance(sampling_params, list):
            sampling_params = [sampling_params] * len(prompts)
        if len(sampling_params) != len(prompts):
            raise ValueError("one SamplingParams per prompt (or a single one for all)")
        ids = [self.add_request(p, sp) for p, sp in zip(prompts, sampling_params)]
        outputs: dict[int, list[int]] = {}
        pbar = None
        if use_tqdm:
            from tqdm.auto import tqdm

            pbar = tqdm(total=len(prompts), desc="Generating", dynamic_ncols=True)
        while not self.is_finished():
            for seq_id, token_ids in self.step():
                outputs[seq_id] = token_ids
                if pbar is not None:
                    pbar.update(1)
        if pbar is not None:
            pbar.close()
        results = []
        for seq_id in ids:
            toks = outputs[seq_id]
            text = self.tokenizer.decode(toks) if self.tokenizer is not None else None
            results.append({"text": text, "token_ids": toks})
        return results

    # ------------------------------------------------------------------ summaries

    def throughput_summary(self) -> dict:
        """Decode / prefill throughput of the last generate() call."""
        dec = [s for s in self.step_stats if not s["prefill"]]
        pre = [s for s in self.step_stats if s["prefill"]]
        dt = sum(s["step_time"] for s in dec)
        pt = sum(s["step_time"] for s in pre)
        return dict(
            decode_steps=len(dec), decode_tokens=sum(s["tokens"] for s in dec), decode_time_s=dt,
            decode_tok_s=(sum(s["tokens"] for s in dec) / dt) if dt else 0.0,
            prefill_steps=len(pre), prefill_tokens=sum(s["tokens"] for s in pre), prefill_time_s=pt,
            prefill_tok_s=(sum(s["tokens"] for s in pre) / pt) if pt else 0.0,
            prefix_cache_hit_tokens=self.scheduler.block_manager.prefix_cache_hit_tokens)


class LLM(LLMEngine):
    """kavor.LLM: the user-facing name of the engine."""
