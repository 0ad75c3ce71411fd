"""The HF generate(custom_generate=...) bridge and the benchmark harness on
the GPU, with a tiny random-init bf16 transformers Llama of head_dim 128
(4 query heads, 1 KV head: GH 4).  santa_flash with a budget that samples
every tile many times must give the exact backend's greedy tokens;
santa_prop must run batched and give finite logits; the harness CLI must
write its files."""
import json
import os

import pytest
import torch

pytest.importorskip("transformers")

pytestmark = pytest.mark.gpu


def _model():
    from santa_amd import harness

    return harness.make_model("tiny", torch.device("cuda:0"), seed=7)


def test_bridge_santa_backends_match_exact_tokens():
    from santa_amd import attention_backends as ab
    from santa_amd import hf_bridge
    from santa_amd.runtime import ExactDecodeBackend

    print("\n[case] hf bridge tiny bf16 model B=2 P=3000 steps=8", flush=True)
    m = _model()
    ids = torch.randint(3, 1000, (2, 3000), generator=torch.Generator().manual_seed(11)).cuda()
    seqs = {}
    for name, backend in (("exact", ExactDecodeBackend()),
                          ("flash", ab.SantaFlashBackend(S=64 * 32 * 32, seed=1690, block_n=None))):
        trace = hf_bridge.HFGenerateTrace()
        seqs[name] = hf_bridge.run_generate_with_hf_custom_loop(model=m, prompt_ids=ids, attention_backend=backend,
                                                                max_new_tokens=8, runtime_trace=trace)
        torch.cuda.synchronize()
        assert trace.steps_sampled == 8 and trace.decode_time_s > 0
    assert torch.equal(seqs["exact"], seqs["flash"])
    prop = ab.SantaPropBackend(S=700, seed=1690, block_n=None)
    out = hf_bridge.run_generate_with_hf_custom_loop(model=m, prompt_ids=ids, attention_backend=prop, max_new_tokens=4)
    torch.cuda.synchronize()
    assert out.shape == (2, 3004) and prop.info()["actual_mode"] == "batch"


def test_harness_cli_writes_its_files(tmp_path):
    from santa_amd import harness

    print("\n[case] harness CLI tiny model B=2 P=2048 new=6", flush=True)
    out = str(tmp_path / "run")
    rc = harness.main(["--out-dir", out, "--model", "tiny", "--batch-size", "2", "--prompt-len", "2048",
                       "--max-new-tokens", "6", "--warmup-runs", "0", "--timed-runs", "1",
                       "--backends", "santa_flash", "santa_prop", "exact"])
    assert rc == 0
    with open(os.path.join(out, "aggregates.json")) as f:
        agg = json.load(f)
    assert set(agg) == {"santa_flash", "santa_prop", "exact_fp32"}
    for payload in agg.values():
        assert payload["metrics"]["output_tokens_per_s"]["mean"] > 0
    with open(os.path.join(out, "backend_agreement.json")) as f:
        assert len(json.load(f)) == 3
