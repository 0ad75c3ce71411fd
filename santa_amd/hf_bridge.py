"""Hugging Face ``generate(custom_generate=...)`` bridge for the sampled-attention decode.

The counterpart of tutorial_code/hf_generate_bridge.py:181-419.  A caller keeps
the Hugging Face surface -- ``model.generate(input_ids, max_new_tokens=...,
custom_generate=loop)`` on a transformers Llama-family causal LM -- and the
decode runs through an attention backend of this package (santa_flash,
santa_prop, or the exact one) over contiguous NHD caches.

What differs from the reference, by design:
- The model is driven through its own modules (embeddings, norms, q/k/v/o
  projections, rotary embedding, MLP, head), never through its attention or
  its cache objects.  The reference converts HF caches to NHD after an HF
  prefill (tutorial_code/runtime_common.py:229-241, 340-397), an API that
  changed in transformers 5; here the prefill writes the NHD caches directly
  (exact causal attention in float32), so nothing depends on HF's cache
  classes.
- Stopping is tracked on the device: in the "fixed" lockstep mode the loop
  never synchronises with the host per step (the reference reads every
  step's tokens back, hf_generate_bridge.py:302-307); "all_finished" checks
  for the end every few steps and trims the extra steps, which only ever hold
  fill tokens, so the returned sequences are the same.

Greedy decoding only, as in the reference (:266-271).
"""
from __future__ import annotations

import inspect
import time
from dataclasses import dataclass, field
from typing import Any, Dict, List, Optional, Sequence

import torch

from .runtime import LlamaShape, NHDCache, causal_attention

__all__ = ["HFGenerateTrace", "HFLlamaRunner", "ensure_hf_custom_generate_available", "resolve_stop_token_ids",
           "resolve_pad_token_id", "resolve_max_new_tokens", "surrogate_pad_token_id",
           "build_hf_custom_generate_loop", "run_generate_with_hf_custom_loop", "split_generated"]


@dataclass
class HFGenerateTrace:
    """Timings and token bookkeeping of one custom generate call (the fields
    of tutorial_code/hf_generate_bridge.py:21-38)."""

    prefill_time_s: float = 0.0
    cache_setup_time_s: float = 0.0
    decode_time_s: float = 0.0
    inner_wall_time_s: float = 0.0
    generate_api_wall_time_s: float = 0.0
    steps_sampled: int = 0
    timed_generated_tokens: int = 0
    visible_generated_tokens: int = 0
    stop_fill_id: Optional[int] = None
    first_stop_step: List[Optional[int]] = field(default_factory=list)
    generated_token_ids_all: List[List[int]] = field(default_factory=list)

    @property
    def end_to_end_wall_time_s(self) -> float:
        return self.generate_api_wall_time_s if self.generate_api_wall_time_s > 0.0 else self.inner_wall_time_s


def ensure_hf_custom_generate_available(model: Any) -> None:
    """Raises when model.generate has no custom_generate hook (hf_generate_bridge.py:41-50)."""
    try:
        params = inspect.signature(model.generate).parameters
    except (TypeError, ValueError) as exc:
        raise RuntimeError("Could not introspect model.generate to verify HF custom_generate support.") from exc
    if "custom_generate" not in params:
        raise RuntimeError("This transformers build does not expose generate(custom_generate=...). "
                           "Please upgrade transformers to a version that supports the official custom_generate hook.")


def _ids(value: Any) -> List[int]:
    if value is None:
        return []
    if isinstance(value, int):
        return [value]
    if isinstance(value, (list, tuple, set)):
        return [int(x) for x in value]
    return []


def _config_chain(model: Any, generation_config: Any) -> List[Any]:
    return [generation_config, getattr(model, "generation_config", None), getattr(model, "config", None)]


def resolve_stop_token_ids(model: Any, generation_config: Any, extra_stop_token_ids: Sequence[int]) -> List[int]:
    """Sorted non-negative ids: the extra ones plus every eos_token_id of the
    generation config, the model's generation config and its config
    (hf_generate_bridge.py:63-72)."""
    ids = set(int(x) for x in extra_stop_token_ids)
    for src in _config_chain(model, generation_config):
        ids.update(_ids(getattr(src, "eos_token_id", None)))
    return sorted(x for x in ids if x >= 0)


def resolve_pad_token_id(model: Any, generation_config: Any, fallback_stop_ids: Sequence[int]) -> int:
    """The first pad_token_id found, else the first stop id, else the first
    eos id, else 0 (hf_generate_bridge.py:75-93)."""
    for src in _config_chain(model, generation_config):
        pad = getattr(src, "pad_token_id", None)
        if pad is not None:
            return int(pad)
    if fallback_stop_ids:
        return int(fallback_stop_ids[0])
    for src in _config_chain(model, generation_config):
        eos = _ids(getattr(src, "eos_token_id", None))
        if eos:
            return eos[0]
    return 0


def resolve_max_new_tokens(input_ids: torch.Tensor, generation_config: Any, stopping_criteria: Optional[Any]) -> int:
    """max_new_tokens of the generation config, else what a max_length
    criterion or the config's max_length leaves after the prompt
    (hf_generate_bridge.py:159-178)."""
    n = getattr(generation_config, "max_new_tokens", None)
    if n is not None:
        return int(n)
    prompt = int(input_ids.shape[1])
    for crit in stopping_criteria or ():
        max_length = getattr(crit, "max_length", None)
        if max_length is not None:
            return max(0, int(max_length) - prompt)
    max_length = getattr(generation_config, "max_length", None)
    if max_length is not None:
        return max(0, int(max_length) - prompt)
    raise ValueError("Could not infer max_new_tokens from generation_config or stopping_criteria.")


def surrogate_pad_token_id(model: Any, prompt_ids: torch.Tensor, preferred: Optional[int],
                           stop_token_ids: Sequence[int]) -> int:
    """A pad id that is neither a stop token nor present in the (unpadded)
    prompts, so that HF infers an all-ones attention mask without warning
    (the purpose of hf_generate_bridge.py:96-156): the preferred id when it is
    not a stop token, else the highest such id of the vocabulary."""
    stops = set(int(x) for x in stop_token_ids)
    if preferred is not None and int(preferred) not in stops:
        return int(preferred)
    vocab = int(getattr(getattr(model, "config", None), "vocab_size", 0) or 0)
    used = set(torch.unique(prompt_ids).tolist()) | stops
    for tok in range(vocab - 1, -1, -1):
        if tok not in used:
            return tok
    if preferred is not None:
        return int(preferred)
    return min(stops) if stops else 0


def _rotate_half(x: torch.Tensor) -> torch.Tensor:
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


class HFLlamaRunner:
    """Prefill and one-token decode of a transformers Llama-family causal LM
    (``model.model.{embed_tokens, layers, norm, rotary_emb}``, ``model.lm_head``;
    each layer with ``input_layernorm``, ``self_attn.{q,k,v,o}_proj``,
    ``post_attention_layernorm``, ``mlp``) over NHD caches, with the attention
    of the decode steps from an attention backend.  The role of the
    reference's forward_one_token_manual_batched
    (tutorial_code/runtime_common.py:501-571)."""

    def __init__(self, model: Any):
        core = model.model
        cfg = model.config
        self.model = model
        self.embed = core.embed_tokens
        self.layers = list(core.layers)
        self.norm = core.norm
        self.rotary = core.rotary_emb
        self.lm_head = model.lm_head
        heads, kv_heads = int(cfg.num_attention_heads), int(cfg.num_key_value_heads)
        hidden = int(cfg.hidden_size)
        head_dim = int(getattr(cfg, "head_dim", None) or hidden // heads)
        if head_dim != hidden // heads:
            raise NotImplementedError(f"head_dim {head_dim} != hidden_size / num_attention_heads ({hidden // heads})")
        self.shape = LlamaShape(hidden=hidden, intermediate=int(cfg.intermediate_size), heads=heads,
                                kv_heads=kv_heads, layers=int(cfg.num_hidden_layers), vocab=int(cfg.vocab_size),
                                rms_eps=float(getattr(cfg, "rms_norm_eps", 1e-5)))
        self.dtype = self.embed.weight.dtype
        self.device = self.embed.weight.device

    def new_cache(self, batch: int, storage: int) -> NHDCache:
        return NHDCache(self.shape, batch, storage, self.dtype, self.device)

    def _rope(self, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
        # x [B, P, heads, D]; cos / sin [B, P, D] from the model's rotary embedding
        return x * cos[:, :, None] + _rotate_half(x) * sin[:, :, None]

    @torch.inference_mode()
    def prefill(self, tokens: torch.Tensor, cache: NHDCache, *, row_chunk: int = 8192,
                attn_chunk: int = 512) -> torch.Tensor:
        """Causal forward over the prompts [B, P]: K/V of positions 0..P-1 into
        the caches, the last position's logits [B, V] (float32) returned."""
        s, D = self.shape, self.shape.head_dim
        B, P = tokens.shape
        h = self.embed(tokens)
        pos = torch.arange(P, device=tokens.device)[None].expand(B, P)
        cos, sin = self.rotary(h, pos)
        for li, layer in enumerate(self.layers):
            attn = layer.self_attn
            x = layer.input_layernorm(h)
            q = self._rope(attn.q_proj(x).view(B, P, s.heads, D), cos, sin)
            k = self._rope(attn.k_proj(x).view(B, P, s.kv_heads, D), cos, sin)
            v = attn.v_proj(x).view(B, P, s.kv_heads, D)
            cache.k[li][:, :P].copy_(k)
            cache.v[li][:, :P].copy_(v)
            a = causal_attention(q, k, v, chunk=attn_chunk)
            del q, k, v, x
            h = h + attn.o_proj(a.reshape(B, P, s.heads * D))
            del a
            for c0 in range(0, P, row_chunk):
                hc = h[:, c0:c0 + row_chunk]
                hc += layer.mlp(layer.post_attention_layernorm(hc))
        return self.lm_head(self.norm(h[:, -1])).float()

    @torch.inference_mode()
    def decode_step(self, token: torch.Tensor, pos: int, cache: NHDCache, backend) -> torch.Tensor:
        """One token per sequence (token [B]) at position pos: cache writes,
        the backend's attention over positions 0..pos, the logits [B, V]."""
        s, D = self.shape, self.shape.head_dim
        B = token.shape[0]
        h = self.embed(token)[:, None]  # [B, 1, hidden]
        cos, sin = self.rotary(h, torch.full((B, 1), pos, dtype=torch.long, device=token.device))
        for li, layer in enumerate(self.layers):
            attn = layer.self_attn
            x = layer.input_layernorm(h)
            q = self._rope(attn.q_proj(x).view(B, 1, s.heads, D), cos, sin)
            k = self._rope(attn.k_proj(x).view(B, 1, s.kv_heads, D), cos, sin)
            v = attn.v_proj(x).view(B, 1, s.kv_heads, D)
            cache.write(li, pos, k[:, 0], v[:, 0])
            a = backend.decode(q[:, 0].contiguous(), cache.k[li], cache.v[li], pos + 1)
            h = h + attn.o_proj(a.reshape(B, 1, s.heads * D))
            h = h + layer.mlp(layer.post_attention_layernorm(h))
        return self.lm_head(self.norm(h[:, 0])).float()


def _sync(device: torch.device) -> None:
    if device.type == "cuda":
        torch.cuda.synchronize(device)


def split_generated(generated: List[List[int]], stop_ids: Sequence[int]) -> List[Optional[int]]:
    """First step at which each sequence emitted a stop token (None if never)."""
    stops = set(int(x) for x in stop_ids)
    out: List[Optional[int]] = []
    for row in generated:
        out.append(next((i for i, t in enumerate(row) if t in stops), None))
    return out


def build_hf_custom_generate_loop(*, attention_backend: Any, prefill_chunk_size: int = 8192,
                                  extra_stop_token_ids: Sequence[int] = (), lockstep_stop_mode: str = "fixed",
                                  runtime_trace: Optional[HFGenerateTrace] = None, stop_check_interval: int = 8):
    """The callable to pass as ``generate(custom_generate=...)``
    (tutorial_code/hf_generate_bridge.py:181-366): greedy lockstep decode
    through attention_backend.  A sequence that emitted a stop token is fed
    the fill token (the first stop id, else the pad id) from then on.
    "fixed" runs max_new_tokens steps; "all_finished" ends once every
    sequence has stopped."""
    if lockstep_stop_mode not in ("fixed", "all_finished"):
        raise ValueError(f"Unsupported lockstep_stop_mode: {lockstep_stop_mode}")
    interval = max(1, int(stop_check_interval))

    @torch.inference_mode()
    def custom_loop(model: Any, input_ids: torch.Tensor, attention_mask: Optional[torch.Tensor] = None,
                    logits_processor: Optional[Any] = None, stopping_criteria: Optional[Any] = None,
                    generation_config: Optional[Any] = None, streamer: Optional[Any] = None,
                    **model_kwargs: Any) -> torch.Tensor:
        # prompts are uniform-length and unpadded; HF's mask and cache objects are not used
        del attention_mask, model_kwargs
        generation_config = generation_config if generation_config is not None else getattr(
            model, "generation_config", None)
        if generation_config is None:
            raise ValueError("generation_config is required for the custom HF generate loop.")
        if input_ids.dim() != 2:
            raise ValueError(f"Expected input_ids rank 2, got shape {tuple(input_ids.shape)}")
        if streamer is not None:
            raise NotImplementedError("Streamer support is not implemented for this custom HF benchmark loop.")
        if bool(getattr(generation_config, "do_sample", False)) or int(getattr(generation_config, "num_beams", 1) or 1) != 1:
            raise NotImplementedError(
                "This custom HF benchmark loop currently supports greedy decoding only (do_sample=False, num_beams=1).")
        B, P = input_ids.shape
        dev = input_ids.device
        max_new = resolve_max_new_tokens(input_ids, generation_config, stopping_criteria)
        stop_ids = resolve_stop_token_ids(model, generation_config, extra_stop_token_ids)
        pad_id = resolve_pad_token_id(model, generation_config, stop_ids)
        fill = int(stop_ids[0]) if stop_ids else int(pad_id)
        use_lp = logits_processor is not None and len(logits_processor) > 0
        runner = HFLlamaRunner(model)

        _sync(dev)
        t_in0 = time.perf_counter()
        t_c0 = time.perf_counter()
        cache = runner.new_cache(B, P + max(max_new, 1))
        _sync(dev)
        t_c1 = time.perf_counter()
        t_p0 = time.perf_counter()
        logits = runner.prefill(input_ids, cache, row_chunk=int(prefill_chunk_size))
        _sync(dev)
        t_p1 = time.perf_counter()

        stop_t = torch.tensor(stop_ids, dtype=torch.long, device=dev)
        finished = torch.zeros(B, dtype=torch.bool, device=dev)
        cur_ids = input_ids if use_lp else None
        toks: List[torch.Tensor] = []
        pos = P
        t_d0 = time.perf_counter()
        for step in range(max_new):
            lg = logits_processor(cur_ids, logits) if use_lp else logits
            nxt = torch.where(finished, torch.full_like(finished, fill, dtype=torch.long), torch.argmax(lg, dim=-1))
            toks.append(nxt)
            finished = finished | torch.isin(nxt, stop_t)
            if use_lp:
                cur_ids = torch.cat((cur_ids, nxt[:, None]), dim=1)
            if step == max_new - 1:
                break
            if lockstep_stop_mode == "all_finished" and (step + 1) % interval == 0 and bool(finished.all()):
                break
            logits = runner.decode_step(nxt, pos, cache, attention_backend)
            pos += 1
        _sync(dev)
        t_d1 = time.perf_counter()

        gen = torch.stack(toks, dim=1) if toks else input_ids.new_zeros(B, 0)
        rows = gen.tolist()
        first_stop = split_generated(rows, stop_ids)
        if lockstep_stop_mode == "all_finished" and rows and all(s is not None for s in first_stop):
            steps = max(first_stop) + 1  # the step at which the last sequence stopped
            rows = [r[:steps] for r in rows]
            gen = gen[:, :steps]
        steps = gen.shape[1]
        sequences = torch.cat((input_ids, gen.to(input_ids.dtype)), dim=1)
        _sync(dev)
        t_in1 = time.perf_counter()
        if runtime_trace is not None:
            runtime_trace.prefill_time_s = t_p1 - t_p0
            runtime_trace.cache_setup_time_s = t_c1 - t_c0
            runtime_trace.decode_time_s = t_d1 - t_d0
            runtime_trace.inner_wall_time_s = t_in1 - t_in0
            runtime_trace.steps_sampled = int(steps)
            runtime_trace.timed_generated_tokens = int(B * steps)
            runtime_trace.visible_generated_tokens = int(
                sum(len(r) if s is None else s for r, s in zip(rows, first_stop)))
            runtime_trace.stop_fill_id = fill
            runtime_trace.first_stop_step = list(first_stop)
            runtime_trace.generated_token_ids_all = [list(r) for r in rows]
        return sequences

    return custom_loop


def run_generate_with_hf_custom_loop(*, model: Any, prompt_ids: torch.Tensor, attention_backend: Any,
                                     max_new_tokens: int, tokenizer: Any = None, prefill_chunk_size: int = 8192,
                                     stop_token_ids: Sequence[int] = (), lockstep_stop_mode: str = "fixed",
                                     runtime_trace: Optional[HFGenerateTrace] = None) -> torch.Tensor:
    """model.generate(...) with the custom loop, greedy, the wall time of the
    whole call into the trace (tutorial_code/hf_generate_bridge.py:369-419)."""
    ensure_hf_custom_generate_available(model)
    trace = runtime_trace if runtime_trace is not None else HFGenerateTrace()
    loop = build_hf_custom_generate_loop(attention_backend=attention_backend, prefill_chunk_size=prefill_chunk_size,
                                         extra_stop_token_ids=list(stop_token_ids),
                                         lockstep_stop_mode=lockstep_stop_mode, runtime_trace=trace)
    _sync(prompt_ids.device)
    t0 = time.perf_counter()
    preferred = getattr(tokenizer, "pad_token_id", None) if tokenizer is not None else None
    pad = surrogate_pad_token_id(model, prompt_ids, preferred,
                                 resolve_stop_token_ids(model, getattr(model, "generation_config", None),
                                                        stop_token_ids))
    sequences = model.generate(input_ids=prompt_ids, do_sample=False, num_beams=1, use_cache=True,
                               max_new_tokens=int(max_new_tokens), pad_token_id=int(pad),
                               return_dict_in_generate=False, custom_generate=loop)
    _sync(prompt_ids.device)
    trace.generate_api_wall_time_s = time.perf_counter() - t0
    return sequences
