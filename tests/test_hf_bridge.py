"""The Hugging Face generate(custom_generate=...) bridge on the CPU.

A tiny random-init transformers LlamaForCausalLM in float32:
- the runner's prefill logits equal the model's own forward;
- decode steps through the exact backend equal the model's forward over the
  whole sequence;
- model.generate(custom_generate=bridge loop) with the exact backend returns
  the same tokens as the model's own greedy generate;
- stop tokens: a sequence that stops is fed the fill token, visible tokens end
  before the stop, and "all_finished" ends at the step where the last
  sequence stopped.
"""
import pytest
import torch

transformers = pytest.importorskip("transformers")

from santa_amd import hf_bridge  # noqa: E402
from santa_amd.runtime import ExactDecodeBackend  # noqa: E402


def tiny_model(seed=3):
    from transformers import LlamaConfig, LlamaForCausalLM

    torch.manual_seed(seed)
    cfg = LlamaConfig(hidden_size=64, intermediate_size=128, num_attention_heads=4, num_key_value_heads=2,
                      num_hidden_layers=2, vocab_size=97, rope_theta=5e5, max_position_embeddings=256,
                      bos_token_id=1, eos_token_id=2, pad_token_id=None)
    m = LlamaForCausalLM(cfg).eval()
    return m


def prompts(B=2, P=13, vocab=97, seed=5):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(3, vocab, (B, P), generator=g)


def test_runner_matches_the_model_forward():
    m = tiny_model()
    ids = prompts()
    runner = hf_bridge.HFLlamaRunner(m)
    cache = runner.new_cache(ids.shape[0], ids.shape[1] + 4)
    lg = runner.prefill(ids, cache)
    with torch.no_grad():
        ref = m(ids).logits[:, -1].float()
    torch.testing.assert_close(lg, ref, atol=1e-4, rtol=1e-4)
    # two decode steps through the exact backend = the model's forward over the longer sequence
    nxt = ids.new_tensor([5, 7])
    lg1 = runner.decode_step(nxt, ids.shape[1], cache, ExactDecodeBackend())
    with torch.no_grad():
        ref1 = m(torch.cat([ids, nxt[:, None]], dim=1)).logits[:, -1].float()
    torch.testing.assert_close(lg1, ref1, atol=1e-4, rtol=1e-4)


def test_custom_generate_matches_hf_greedy():
    m = tiny_model()
    ids = prompts()
    trace = hf_bridge.HFGenerateTrace()
    seq = hf_bridge.run_generate_with_hf_custom_loop(model=m, prompt_ids=ids, attention_backend=ExactDecodeBackend(),
                                                     max_new_tokens=10, runtime_trace=trace)
    with torch.no_grad():
        ref = m.generate(input_ids=ids, do_sample=False, num_beams=1, max_new_tokens=10, eos_token_id=[],
                         pad_token_id=0)
    # HF stops a row at eos (2); compare up to the first stop of either
    first = hf_bridge.split_generated(seq[:, ids.shape[1]:].tolist(), [2])
    for b in range(ids.shape[0]):
        n = 10 if first[b] is None else first[b] + 1
        assert seq[b, ids.shape[1]:ids.shape[1] + n].tolist() == ref[b, ids.shape[1]:ids.shape[1] + n].tolist()
    assert trace.steps_sampled == 10 and trace.timed_generated_tokens == 20
    assert trace.generate_api_wall_time_s > 0 and trace.decode_time_s > 0 and trace.prefill_time_s > 0
    assert len(trace.generated_token_ids_all) == 2 and all(len(r) == 10 for r in trace.generated_token_ids_all)


def test_stop_tokens_fill_and_all_finished():
    m = tiny_model()
    ids = prompts()
    # the free-running tokens, to pick stop ids that occur
    free = hf_bridge.run_generate_with_hf_custom_loop(model=m, prompt_ids=ids, attention_backend=ExactDecodeBackend(),
                                                      max_new_tokens=12)[:, ids.shape[1]:].tolist()
    stop_a, stop_b = free[0][1], free[1][3]
    trace = hf_bridge.HFGenerateTrace()
    loop = hf_bridge.build_hf_custom_generate_loop(attention_backend=ExactDecodeBackend(),
                                                   extra_stop_token_ids=[stop_a, stop_b],
                                                   lockstep_stop_mode="all_finished", runtime_trace=trace,
                                                   stop_check_interval=3)
    seq = m.generate(input_ids=ids, do_sample=False, num_beams=1, max_new_tokens=12, pad_token_id=0,
                     custom_generate=loop)
    gen = seq[:, ids.shape[1]:].tolist()
    first = trace.first_stop_step
    assert first[0] is not None and first[0] <= 1 and first[1] is not None and first[1] <= 3
    assert trace.steps_sampled == max(first) + 1 == len(gen[0])
    fill = trace.stop_fill_id
    assert fill == min(set([stop_a, stop_b, 2]))
    for b in range(2):
        assert all(t == fill for t in gen[b][first[b] + 1:])
    assert trace.visible_generated_tokens == first[0] + first[1]
