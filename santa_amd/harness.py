"""Long-context decode benchmark with the reference's output files.

The counterpart of tutorial_code/benchmark_longctx.py: for every backend and
run it decodes every batch, then writes into the output directory the files
the reference's consumers read (same names, keys and statistics):

- ``batch_metrics.jsonl``: one row per (phase, run, backend, batch)
  (benchmark_longctx.py:350-369, 604-611);
- ``generations.jsonl``: one row per generated sequence (:371-391, 614-621);
- ``run_metrics.jsonl``: the batches of one (phase, run, backend) aggregated
  (:396-426, 634-645);
- ``aggregates.json`` / ``aggregates.csv``: per backend, summary statistics of
  the timed runs (:656-686, 486-530);
- ``backend_agreement.json``: pairwise token / text agreement (:429-483);
- ``config.json``, ``dataset_summary.json``, ``examples_used.jsonl``.

What it runs on is synthetic, since there is no network for checkpoints or
datasets: a random-init transformers Llama-family model (N(0, 0.02) weights,
transformers' initialisation) and seeded random prompt tokens of one length.
With no tokenizer, "text" fields hold the token ids joined by spaces and
exact match is false (the prompts have no reference answers).  The decode goes
through HFLlamaRunner (hf_bridge) with the attention backends of this package,
either directly ("manual" surface) or through
``model.generate(custom_generate=...)`` ("hf_generate").

    python -m santa_amd.harness --out-dir runs/x --model llama-3.1-8b \\
        --batch-size 4 --prompt-len 32768 --num-batches 1 --max-new-tokens 64 \\
        --backends santa_flash santa_prop exact
"""
from __future__ import annotations

import argparse
import csv
import json
import math
import os
import statistics
import time
from collections import defaultdict
from dataclasses import dataclass
from typing import Any, Dict, Iterable, List, Optional, Sequence, Tuple

import torch

from . import hf_bridge

METRICS_TO_SUMMARIZE = ["prefill_time_s", "cache_setup_time_s", "decode_time_s", "end_to_end_wall_time_s", "tpot_ms",
                        "output_tokens_per_s", "visible_output_tokens_per_s", "requests_per_s",
                        "prefill_tokens_per_s", "exact_match_rate"]


# ------------------------------------------------------------------ files
def write_json(path: str, payload: Any) -> None:
    with open(path, "w", encoding="utf-8") as f:
        json.dump(payload, f, indent=2, ensure_ascii=False)


def write_jsonl(path: str, rows: Iterable[Dict[str, Any]]) -> None:
    with open(path, "w", encoding="utf-8") as f:
        for row in rows:
            f.write(json.dumps(row, ensure_ascii=False) + "\n")


def flatten_backend_info(prefix: str, info: Dict[str, Any]) -> Dict[str, Any]:
    return {f"{prefix}{k}": v for k, v in info.items()}


# ------------------------------------------------------------------ statistics
def _quantile(values: Sequence[float], q: float) -> float:
    """Linear interpolation between order statistics (runtime_common.py:449-462)."""
    if not values:
        return float("nan")
    v = sorted(float(x) for x in values)
    x = (len(v) - 1) * q
    lo, hi = math.floor(x), math.ceil(x)
    return v[lo] if lo == hi else v[lo] + (v[hi] - v[lo]) * (x - lo)


def summarize_numeric(values: Sequence[float]) -> Dict[str, float]:
    """count, mean, std (sample), median, p90, min, max and a normal 95 %
    interval of the mean (runtime_common.py:465-496)."""
    vals = [float(v) for v in values]
    if not vals:
        nan = float("nan")
        return {"count": 0, "mean": nan, "std": nan, "median": nan, "p90": nan, "min": nan, "max": nan,
                "ci95_lo": nan, "ci95_hi": nan}
    mean = statistics.fmean(vals)
    std = statistics.stdev(vals) if len(vals) > 1 else 0.0
    hw = 1.96 * std / math.sqrt(len(vals)) if len(vals) > 1 else 0.0
    return {"count": len(vals), "mean": mean, "std": std, "median": _quantile(vals, 0.5), "p90": _quantile(vals, 0.9),
            "min": min(vals), "max": max(vals), "ci95_lo": mean - hw, "ci95_hi": mean + hw}


def _ratio(a: float, b: float) -> float:
    return a / b if b > 0 else float("nan")


def batch_metric_row(*, batch_id: int, batch_size: int, example_indices: Sequence[int], prompt_len: int,
                     prefill_time_s: float, cache_setup_time_s: float, decode_time_s: float,
                     generate_api_wall_time_s: float, end_to_end_wall_time_s: float, timed_generated_tokens: int,
                     visible_generated_tokens: int) -> Dict[str, Any]:
    """The per-batch metric row (benchmark_longctx.py:347-369)."""
    return {
        "batch_id": int(batch_id),
        "batch_size": int(batch_size),
        "example_indices": list(example_indices),
        "prompt_len": int(prompt_len),
        "prefill_time_s": float(prefill_time_s),
        "cache_setup_time_s": float(cache_setup_time_s),
        "decode_time_s": float(decode_time_s),
        "generate_api_wall_time_s": float(generate_api_wall_time_s),
        "hf_generate_wrapper_overhead_s": float(end_to_end_wall_time_s
                                                 - (prefill_time_s + cache_setup_time_s + decode_time_s)),
        "end_to_end_wall_time_s": float(end_to_end_wall_time_s),
        "timed_generated_tokens": int(timed_generated_tokens),
        "visible_generated_tokens": int(visible_generated_tokens),
        "steps_sampled": int(timed_generated_tokens // batch_size) if batch_size > 0 else 0,
        "tpot_ms": 1000.0 * _ratio(decode_time_s, timed_generated_tokens),
        "output_tokens_per_s": _ratio(timed_generated_tokens, decode_time_s),
        "visible_output_tokens_per_s": _ratio(visible_generated_tokens, decode_time_s),
        "requests_per_s": _ratio(batch_size, end_to_end_wall_time_s),
        "prefill_tokens_per_s": _ratio(batch_size * prompt_len, prefill_time_s),
    }


def aggregate_run_rows(batch_rows: Sequence[Dict[str, Any]], generation_rows: Sequence[Dict[str, Any]]) -> Dict[str, Any]:
    """Sums over a run's batches and the rates they give (benchmark_longctx.py:396-426)."""
    tot = lambda key, kind=float: kind(sum(kind(r[key]) for r in batch_rows))  # noqa: E731
    out: Dict[str, Any] = {
        "num_batches": len(batch_rows),
        "num_requests": tot("batch_size", int),
        "prefill_time_s": tot("prefill_time_s"),
        "cache_setup_time_s": tot("cache_setup_time_s"),
        "decode_time_s": tot("decode_time_s"),
        "end_to_end_wall_time_s": tot("end_to_end_wall_time_s"),
        "timed_generated_tokens": tot("timed_generated_tokens", int),
        "visible_generated_tokens": tot("visible_generated_tokens", int),
        "prompt_tokens_total": int(sum(int(r["batch_size"]) * int(r["prompt_len"]) for r in batch_rows)),
    }
    out["tpot_ms"] = 1000.0 * _ratio(out["decode_time_s"], out["timed_generated_tokens"])
    out["output_tokens_per_s"] = _ratio(out["timed_generated_tokens"], out["decode_time_s"])
    out["visible_output_tokens_per_s"] = _ratio(out["visible_generated_tokens"], out["decode_time_s"])
    out["requests_per_s"] = _ratio(out["num_requests"], out["end_to_end_wall_time_s"])
    out["prefill_tokens_per_s"] = _ratio(out["prompt_tokens_total"], out["prefill_time_s"])
    out["exact_match_rate"] = (sum(1 for r in generation_rows if bool(r["exact_match"])) / len(generation_rows)
                               if generation_rows else float("nan"))
    return out


def compute_pairwise_agreement(generation_rows: Sequence[Dict[str, Any]]) -> List[Dict[str, Any]]:
    """For every pair of backends, over the (run, example) pairs both decoded:
    normalized-text and visible-token agreement and the exact-match split
    (benchmark_longctx.py:429-483)."""
    rows = {(int(r["run_idx"]), int(r["example_index"]), str(r["backend"])): r for r in generation_rows}
    backends = sorted({str(r["backend"]) for r in generation_rows})
    keys = sorted({(int(r["run_idx"]), int(r["example_index"])) for r in generation_rows})
    out: List[Dict[str, Any]] = []
    for i, a in enumerate(backends):
        for b in backends[i + 1:]:
            n = text = tok = both = a_only = b_only = 0
            for run_idx, ex in keys:
                ra, rb = rows.get((run_idx, ex, a)), rows.get((run_idx, ex, b))
                if ra is None or rb is None:
                    continue
                n += 1
                text += ra["generated_text_normalized"] == rb["generated_text_normalized"]
                tok += ra["generated_token_ids_visible"] == rb["generated_token_ids_visible"]
                ea, eb = bool(ra["exact_match"]), bool(rb["exact_match"])
                both += ea and eb
                a_only += ea and not eb
                b_only += eb and not ea
            if n:
                out.append({"backend_a": a, "backend_b": b, "comparable_examples": n,
                            "normalized_text_match_rate": text / n, "visible_token_id_match_rate": tok / n,
                            "both_exact_match_rate": both / n, "a_only_exact_match_rate": a_only / n,
                            "b_only_exact_match_rate": b_only / n})
    return out


CSV_FIELDS = ["backend", "runs"] + [f"{m}_{s}" for s in ("mean", "median") for m in (
    "prefill_time_s", "decode_time_s", "end_to_end_wall_time_s", "tpot_ms", "output_tokens_per_s", "requests_per_s",
    "exact_match_rate")]


def save_aggregate_csv(path: str, aggregate_payload: Dict[str, Any]) -> None:
    """One row per backend: run count, then means and medians of seven
    metrics (benchmark_longctx.py:486-530)."""
    with open(path, "w", encoding="utf-8", newline="") as f:
        w = csv.DictWriter(f, fieldnames=CSV_FIELDS)
        w.writeheader()
        for backend, payload in aggregate_payload.items():
            row = {"backend": backend, "runs": payload["num_runs"]}
            for field in CSV_FIELDS[2:]:
                metric, stat = field.rsplit("_", 1)
                row[field] = payload["metrics"][metric][stat]
            w.writerow(row)


def aggregate_timed_runs(run_rows: Sequence[Dict[str, Any]]) -> Dict[str, Any]:
    """aggregates.json: per backend, statistics of the timed runs' metrics and
    the last run's backend info (benchmark_longctx.py:656-686)."""
    by_backend: Dict[str, List[Dict[str, Any]]] = defaultdict(list)
    for r in run_rows:
        if r["phase"] == "timed":
            by_backend[str(r["backend"])].append(r)
    return {b: {"num_runs": len(rs),
                "metrics": {m: summarize_numeric([float(r[m]) for r in rs]) for m in METRICS_TO_SUMMARIZE},
                "last_backend_info": {k: v for k, v in rs[-1].items() if k.startswith("backend_")}}
            for b, rs in by_backend.items()}


# ------------------------------------------------------------------ workload
@dataclass
class Batch:
    batch_id: int
    example_indices: List[int]
    prompt_ids: torch.Tensor  # [B, P] on the device


def synthetic_batches(*, num_batches: int, batch_size: int, prompt_len: int, vocab: int, seed: int,
                      device) -> List[Batch]:
    g = torch.Generator().manual_seed(seed)
    out = []
    for i in range(num_batches):
        ids = torch.randint(3, vocab, (batch_size, prompt_len), generator=g)
        out.append(Batch(i, list(range(i * batch_size, (i + 1) * batch_size)), ids.to(device)))
    return out


def _text(ids: Sequence[int], tokenizer: Any) -> str:
    if tokenizer is not None:
        return tokenizer.decode(list(ids))
    return " ".join(str(int(t)) for t in ids)


def run_backend_on_batch(*, model: Any, batch: Batch, backend: Any, max_new_tokens: int, stop_token_ids: Sequence[int],
                         lockstep_stop_mode: str, generation_surface: str, prefill_chunk_size: int,
                         tokenizer: Any = None) -> Tuple[Dict[str, Any], List[Dict[str, Any]]]:
    """Decode one batch with one backend: the batch metric row and one
    generation row per sequence (benchmark_longctx.py:245-393)."""
    trace = hf_bridge.HFGenerateTrace()
    if generation_surface == "hf_generate":
        hf_bridge.run_generate_with_hf_custom_loop(model=model, prompt_ids=batch.prompt_ids, attention_backend=backend,
                                                   max_new_tokens=max_new_tokens, tokenizer=tokenizer,
                                                   prefill_chunk_size=prefill_chunk_size,
                                                   stop_token_ids=stop_token_ids,
                                                   lockstep_stop_mode=lockstep_stop_mode, runtime_trace=trace)
    elif generation_surface == "manual":
        loop = hf_bridge.build_hf_custom_generate_loop(attention_backend=backend,
                                                       prefill_chunk_size=prefill_chunk_size,
                                                       extra_stop_token_ids=stop_token_ids,
                                                       lockstep_stop_mode=lockstep_stop_mode, runtime_trace=trace)
        from transformers import GenerationConfig

        cfg = GenerationConfig(max_new_tokens=int(max_new_tokens), do_sample=False, num_beams=1,
                               eos_token_id=getattr(model.generation_config, "eos_token_id", None))
        t0 = time.perf_counter()
        loop(model, batch.prompt_ids, generation_config=cfg)
        trace.generate_api_wall_time_s = 0.0
        trace.inner_wall_time_s = max(trace.inner_wall_time_s, time.perf_counter() - t0)
    else:
        raise ValueError(f"Unsupported generation_surface: {generation_surface}")
    B, P = batch.prompt_ids.shape
    metric = batch_metric_row(batch_id=batch.batch_id, batch_size=B, example_indices=batch.example_indices,
                              prompt_len=P, prefill_time_s=trace.prefill_time_s,
                              cache_setup_time_s=trace.cache_setup_time_s, decode_time_s=trace.decode_time_s,
                              generate_api_wall_time_s=trace.generate_api_wall_time_s,
                              end_to_end_wall_time_s=trace.end_to_end_wall_time_s,
                              timed_generated_tokens=trace.timed_generated_tokens,
                              visible_generated_tokens=trace.visible_generated_tokens)
    gens = []
    for slot, (ex, ids, stop) in enumerate(zip(batch.example_indices, trace.generated_token_ids_all,
                                               trace.first_stop_step)):
        visible = ids if stop is None else ids[:stop]
        text = _text(visible, tokenizer)
        gens.append({"batch_id": batch.batch_id, "batch_slot": slot, "batch_size": B, "example_index": ex,
                     "prompt_len": P, "original_prompt_len": P, "outputs": [], "answer_prefix": "",
                     "generated_token_ids_all": list(ids), "generated_token_ids_visible": list(visible),
                     "generated_text": text, "generated_text_normalized": text.strip(), "stop_step": stop,
                     "exact_match": False})
    return metric, gens


def run_benchmark(*, model: Any, backends: Sequence[Any], batches: Sequence[Batch], out_dir: str, max_new_tokens: int,
                  warmup_runs: int = 1, timed_runs: int = 1, stop_token_ids: Sequence[int] = (),
                  lockstep_stop_mode: str = "fixed", generation_surface: str = "hf_generate",
                  prefill_chunk_size: int = 8192, config: Optional[Dict[str, Any]] = None, tokenizer: Any = None,
                  log=print) -> Dict[str, Any]:
    """Warm-up and timed runs of every backend over every batch; writes the
    output files and returns the aggregates (benchmark_longctx.py:587-723)."""
    os.makedirs(out_dir, exist_ok=True)
    batch_rows: List[Dict[str, Any]] = []
    gen_rows: List[Dict[str, Any]] = []
    run_rows: List[Dict[str, Any]] = []
    for phase, n_runs in (("warmup", warmup_runs), ("timed", timed_runs)):
        for run_idx in range(n_runs):
            for backend in backends:
                per_batch, per_gen = [], []
                for batch in batches:
                    metric, gens = run_backend_on_batch(model=model, batch=batch, backend=backend,
                                                        max_new_tokens=max_new_tokens, stop_token_ids=stop_token_ids,
                                                        lockstep_stop_mode=lockstep_stop_mode,
                                                        generation_surface=generation_surface,
                                                        prefill_chunk_size=prefill_chunk_size, tokenizer=tokenizer)
                    head = {"phase": phase, "run_idx": run_idx, "backend": backend.name,
                            **flatten_backend_info("backend_", backend.info())}
                    row = {**head, **metric}
                    per_batch.append(row)
                    per_gen.extend({**head, **g} for g in gens)
                    log(f"[{phase} run {run_idx}] backend={backend.name:<12} batch={batch.batch_id:03d} "
                        f"prefill={row['prefill_time_s']:.3f}s decode={row['decode_time_s']:.3f}s "
                        f"TPOT={row['tpot_ms']:.3f} ms")
                batch_rows.extend(per_batch)
                gen_rows.extend(per_gen)
                summary = aggregate_run_rows(per_batch, per_gen)
                summary.update({"phase": phase, "run_idx": run_idx, "backend": backend.name,
                                **flatten_backend_info("backend_", backend.info())})
                run_rows.append(summary)
    write_jsonl(os.path.join(out_dir, "batch_metrics.jsonl"), batch_rows)
    write_jsonl(os.path.join(out_dir, "run_metrics.jsonl"), run_rows)
    write_jsonl(os.path.join(out_dir, "generations.jsonl"), gen_rows)
    aggregates = aggregate_timed_runs(run_rows)
    write_json(os.path.join(out_dir, "aggregates.json"), aggregates)
    save_aggregate_csv(os.path.join(out_dir, "aggregates.csv"), aggregates)
    write_json(os.path.join(out_dir, "backend_agreement.json"),
               compute_pairwise_agreement([r for r in gen_rows if r["phase"] == "timed"]))
    write_json(os.path.join(out_dir, "config.json"), dict(config or {}))
    n = sum(int(b.prompt_ids.shape[0]) for b in batches)
    write_json(os.path.join(out_dir, "dataset_summary.json"),
               {"dataset": "synthetic (seeded random token ids)", "num_examples": n, "dropped_tail_examples": 0})
    write_jsonl(os.path.join(out_dir, "examples_used.jsonl"),
                [{"index": i, "prompt_len": int(b.prompt_ids.shape[1])} for b in batches for i in b.example_indices])
    return aggregates


# ------------------------------------------------------------------ CLI
MODELS = {
    # LlamaConfig of Llama-3.1-8B (the cfg4 shape) and a small one for quick runs
    "llama-3.1-8b": dict(hidden_size=4096, intermediate_size=14336, num_attention_heads=32, num_key_value_heads=8,
                         num_hidden_layers=32, vocab_size=128256, rope_theta=5e5, max_position_embeddings=131072),
    "tiny": dict(hidden_size=512, intermediate_size=1024, num_attention_heads=4, num_key_value_heads=1,
                 num_hidden_layers=2, vocab_size=1000, rope_theta=5e5, max_position_embeddings=131072),
}


def make_model(name: str, device, dtype=torch.bfloat16, seed: int = 1690):
    """A random-init transformers LlamaForCausalLM (weights N(0, 0.02)) on the device."""
    from transformers import LlamaConfig, LlamaForCausalLM

    torch.manual_seed(seed)
    cfg = LlamaConfig(**MODELS[name], bos_token_id=1, eos_token_id=2)
    with torch.device(device):
        model = LlamaForCausalLM(cfg).to(dtype)
    return model.eval()


def build(names: Sequence[str], *, santa_s: int, santa_seed: int, santa_block_n: Optional[int]) -> List[Any]:
    from . import attention_backends as ab
    from .runtime import ExactDecodeBackend

    out = []
    for n in names:
        if n == "santa_flash":
            out.append(ab.SantaFlashBackend(S=santa_s, seed=santa_seed, block_n=santa_block_n))
        elif n == "santa_prop":
            out.append(ab.SantaPropBackend(S=santa_s, seed=santa_seed, block_n=santa_block_n))
        elif n == "exact":
            b = ExactDecodeBackend()
            out.append(b)
        else:
            raise ValueError(f"unknown backend {n!r} (santa_flash, santa_prop, exact)")
    return out


# The backends a run compares by default: the exact comparator (this build's
# counterpart of the reference's FA2 baseline, which is not available on
# ROCm offline) and the two santa variants (benchmark_longctx.py:37).
MAIN_BACKENDS = ["exact", "santa_flash", "santa_prop"]


def format_optional_int(x: Optional[int]) -> str:
    """None -> "unset(default)", else the integer as text (runtime_common.py:99-102)."""
    return "unset(default)" if x is None else str(int(x))


def write_invocation(out_dir: str, args: argparse.Namespace, device: Any, dtype: str = "bf16") -> str:
    """invocation.json: the command-line arguments, device, dtype, santa block
    size and the main backends, written before the model loads
    (benchmark_longctx.py:739-751).  Returns the file's path."""
    os.makedirs(out_dir, exist_ok=True)
    path = os.path.join(out_dir, "invocation.json")
    write_json(path, {"argv": vars(args), "device": str(device), "dtype": dtype,
                      "santa_block_n": format_optional_int(getattr(args, "santa_block_n", None)),
                      "paper_main_backends": list(MAIN_BACKENDS), "timestamp_unix": time.time()})
    return path


def parse_args(argv=None) -> argparse.Namespace:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--out-dir", required=True)
    ap.add_argument("--model", choices=sorted(MODELS), default="tiny")
    ap.add_argument("--backends", nargs="+", default=["santa_flash", "santa_prop", "exact"])
    ap.add_argument("--batch-size", type=int, default=2)
    ap.add_argument("--num-batches", type=int, default=1)
    ap.add_argument("--prompt-len", type=int, default=4096)
    ap.add_argument("--max-new-tokens", type=int, default=16)
    ap.add_argument("--warmup-runs", type=int, default=1)
    ap.add_argument("--timed-runs", type=int, default=1)
    ap.add_argument("--santa-s", type=int, default=256)
    ap.add_argument("--santa-seed", type=int, default=1690)
    ap.add_argument("--santa-block-n", type=int, default=None)
    ap.add_argument("--lockstep-stop-mode", choices=("fixed", "all_finished"), default="fixed")
    ap.add_argument("--generation-surface", choices=("hf_generate", "manual"), default="hf_generate")
    ap.add_argument("--prefill-chunk-size", type=int, default=8192)
    ap.add_argument("--seed", type=int, default=1690)
    return ap.parse_args(argv)


def main(argv=None) -> int:
    args = parse_args(argv)
    dev = torch.device("cuda:0")
    write_invocation(args.out_dir, args, dev)
    model = make_model(args.model, dev, seed=args.seed)
    backends = build(args.backends, santa_s=args.santa_s, santa_seed=args.santa_seed, santa_block_n=args.santa_block_n)
    batches = synthetic_batches(num_batches=args.num_batches, batch_size=args.batch_size, prompt_len=args.prompt_len,
                                vocab=model.config.vocab_size, seed=args.seed, device=dev)
    config = {**vars(args), "dtype": "bf16", "device": str(dev), "model_config": MODELS[args.model],
              "weights": "random N(0, 0.02)"}
    agg = run_benchmark(model=model, backends=backends, batches=batches, out_dir=args.out_dir,
                        max_new_tokens=args.max_new_tokens, warmup_runs=args.warmup_runs, timed_runs=args.timed_runs,
                        lockstep_stop_mode=args.lockstep_stop_mode, generation_surface=args.generation_surface,
                        prefill_chunk_size=args.prefill_chunk_size, config=config)
    for b, p in agg.items():
        m = p["metrics"]
        print(f"{b:<12} output_tok/s={m['output_tokens_per_s']['mean']:.2f} tpot_ms={m['tpot_ms']['mean']:.3f}")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
