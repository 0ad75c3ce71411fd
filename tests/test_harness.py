"""The benchmark harness writes the reference's output files
(tutorial_code/benchmark_longctx.py:347-723) with the same keys; checked on
the CPU with a tiny float32 model and two exact backends, plus closed forms
of the aggregation and statistics."""
import csv
import json
import math
import os

import pytest
import torch

pytest.importorskip("transformers")

from santa_amd import harness  # noqa: E402
from santa_amd.runtime import ExactDecodeBackend  # noqa: E402
from test_hf_bridge import tiny_model  # noqa: E402

BATCH_KEYS = {"phase", "run_idx", "backend", "batch_id", "batch_size", "example_indices", "prompt_len",
              "prefill_time_s", "cache_setup_time_s", "decode_time_s", "generate_api_wall_time_s",
              "hf_generate_wrapper_overhead_s", "end_to_end_wall_time_s", "timed_generated_tokens",
              "visible_generated_tokens", "steps_sampled", "tpot_ms", "output_tokens_per_s",
              "visible_output_tokens_per_s", "requests_per_s", "prefill_tokens_per_s"}
GEN_KEYS = {"phase", "run_idx", "backend", "batch_id", "batch_slot", "batch_size", "example_index", "prompt_len",
            "original_prompt_len", "outputs", "answer_prefix", "generated_token_ids_all",
            "generated_token_ids_visible", "generated_text", "generated_text_normalized", "stop_step", "exact_match"}
RUN_KEYS = {"num_batches", "num_requests", "prefill_time_s", "cache_setup_time_s", "decode_time_s",
            "end_to_end_wall_time_s", "timed_generated_tokens", "visible_generated_tokens", "prompt_tokens_total",
            "tpot_ms", "output_tokens_per_s", "visible_output_tokens_per_s", "requests_per_s", "prefill_tokens_per_s",
            "exact_match_rate", "phase", "run_idx", "backend"}


class ExactTwin(ExactDecodeBackend):
    name = "exact_twin"


def read_jsonl(p):
    with open(p) as f:
        return [json.loads(l) for l in f]


@pytest.mark.parametrize("surface", ["hf_generate", "manual"])
def test_output_files(tmp_path, surface):
    m = tiny_model()
    batches = harness.synthetic_batches(num_batches=2, batch_size=2, prompt_len=11, vocab=97, seed=4, device="cpu")
    out = str(tmp_path / surface)
    agg = harness.run_benchmark(model=m, backends=[ExactDecodeBackend(), ExactTwin()], batches=batches, out_dir=out,
                                max_new_tokens=5, warmup_runs=1, timed_runs=2, generation_surface=surface,
                                config={"k": 1}, log=lambda *_: None)
    names = {"batch_metrics.jsonl", "run_metrics.jsonl", "generations.jsonl", "aggregates.json", "aggregates.csv",
             "backend_agreement.json", "config.json", "dataset_summary.json", "examples_used.jsonl"}
    assert names <= set(os.listdir(out))
    br = read_jsonl(os.path.join(out, "batch_metrics.jsonl"))
    assert len(br) == 3 * 2 * 2  # (1 warm-up + 2 timed runs) x 2 backends x 2 batches
    for r in br:
        assert BATCH_KEYS <= set(r), BATCH_KEYS - set(r)
        assert r["timed_generated_tokens"] == 10 and r["steps_sampled"] == 5
        assert math.isclose(r["tpot_ms"], 1000 * r["decode_time_s"] / 10)
        assert {"backend_backend", "backend_exact_attention"} <= set(r)
    gr = read_jsonl(os.path.join(out, "generations.jsonl"))
    assert len(gr) == 3 * 2 * 4 and all(GEN_KEYS <= set(r) for r in gr)
    rr = read_jsonl(os.path.join(out, "run_metrics.jsonl"))
    assert len(rr) == 3 * 2 and all(RUN_KEYS <= set(r) for r in rr)
    r0 = rr[0]
    rows0 = [r for r in br if r["phase"] == r0["phase"] and r["run_idx"] == r0["run_idx"] and
             r["backend"] == r0["backend"]]
    assert math.isclose(r0["decode_time_s"], sum(r["decode_time_s"] for r in rows0))
    assert r0["prompt_tokens_total"] == 2 * 2 * 11 and r0["num_requests"] == 4
    with open(os.path.join(out, "aggregates.json")) as f:
        agg_file = json.load(f)
    assert set(agg_file) == {"exact_fp32", "exact_twin"} and agg_file["exact_fp32"]["num_runs"] == 2
    stats = agg_file["exact_fp32"]["metrics"]["decode_time_s"]
    assert set(stats) == {"count", "mean", "std", "median", "p90", "min", "max", "ci95_lo", "ci95_hi"}
    assert set(agg_file["exact_fp32"]["metrics"]) == set(harness.METRICS_TO_SUMMARIZE)
    with open(os.path.join(out, "aggregates.csv")) as f:
        rows = list(csv.DictReader(f))
    assert [r["backend"] for r in rows] == ["exact_fp32", "exact_twin"] and list(rows[0]) == harness.CSV_FIELDS
    with open(os.path.join(out, "backend_agreement.json")) as f:
        pairs = json.load(f)
    # the two backends compute the same thing: every token agrees
    assert len(pairs) == 1 and pairs[0]["comparable_examples"] == 2 * 4
    assert pairs[0]["visible_token_id_match_rate"] == 1.0 and pairs[0]["normalized_text_match_rate"] == 1.0
    assert agg is not None


def test_statistics_closed_forms():
    s = harness.summarize_numeric([1.0, 2.0, 3.0, 4.0])
    assert s["count"] == 4 and s["mean"] == 2.5 and s["median"] == 2.5 and s["min"] == 1 and s["max"] == 4
    assert math.isclose(s["std"], math.sqrt(5 / 3)) and math.isclose(s["p90"], 3.7)
    assert math.isclose(s["ci95_hi"] - s["mean"], 1.96 * math.sqrt(5 / 3) / 2)
    one = harness.summarize_numeric([7.0])
    assert one["std"] == 0.0 and one["ci95_lo"] == one["ci95_hi"] == 7.0
    assert math.isnan(harness.summarize_numeric([])["mean"])
    row = harness.batch_metric_row(batch_id=0, batch_size=4, example_indices=[0, 1, 2, 3], prompt_len=100,
                                   prefill_time_s=2.0, cache_setup_time_s=0.5, decode_time_s=4.0,
                                   generate_api_wall_time_s=7.0, end_to_end_wall_time_s=7.0,
                                   timed_generated_tokens=64, visible_generated_tokens=60)
    assert row["tpot_ms"] == 62.5 and row["output_tokens_per_s"] == 16 and row["steps_sampled"] == 16
    assert row["prefill_tokens_per_s"] == 200 and row["hf_generate_wrapper_overhead_s"] == 0.5
    assert math.isclose(row["requests_per_s"], 4 / 7)


def test_invocation_file(tmp_path):
    """invocation.json (tutorial_code/benchmark_longctx.py:739-751): the CLI's
    arguments, device, dtype, block size as text and the main backends."""
    args = harness.parse_args(["--out-dir", str(tmp_path / "inv"), "--santa-block-n", "256"])
    path = harness.write_invocation(args.out_dir, args, torch.device("cpu"))
    with open(path) as f:
        inv = json.load(f)
    assert set(inv) == {"argv", "device", "dtype", "santa_block_n", "paper_main_backends", "timestamp_unix"}
    assert inv["argv"]["santa_block_n"] == 256 and inv["santa_block_n"] == "256"
    assert inv["device"] == "cpu" and inv["dtype"] == "bf16"
    assert inv["paper_main_backends"] == ["exact", "santa_flash", "santa_prop"]
    args = harness.parse_args(["--out-dir", str(tmp_path / "inv2")])
    with open(harness.write_invocation(args.out_dir, args, "cuda:0")) as f:
        assert json.load(f)["santa_block_n"] == "unset(default)"
