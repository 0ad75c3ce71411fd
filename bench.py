#!/usr/bin/env python3
"""Headline benchmark: santa_flash sampled-attention decode on one MI355X.

Workload: Llama-3.1-8B attention shape, batch 8,
32 query / 8 KV heads, head_dim 128, bf16, 32768 cached tokens per sequence,
K/V ~ N(0,1) plus a per-head rank-4 key bias (scale 0.5), S = 256, seed 1690.
One step = one single-layer decode call (santa_flash_batch_cuda.
decode_systematic_batched) over inputs already resident in HBM.

Timing.  The warm-up runs --warmup calls and then keeps calling until at
least --warmup-ms of wall time has passed (the GPU's clocks settle), whatever
--warmup says.  Then exactly --steps calls are timed in one window between
HIP events on torch's current stream (the stream every launch goes on),
bracketed by device synchronisations: ms_per_step and value come from that
window.  Then windows of the whole step and of the dominant kernel alone
(the flash tile pass, the step minus its merge launch) alternate, several of
each, and their medians give kernel_us and us_per_step_median: the tile pass
is part of the step, so kernel_us <= us_per_step_median.

Prints ONE JSON line.  `value` is tokens/s = B / t_step; `roofline.achieved`
is the algorithmic HBM bytes (all valid K rows + emitted V rows + q + out +
m_star) over the tile pass's median duration; `roofline.step_frac` uses the
whole step instead.  `cpu_baseline` is the vectorized PyTorch CPU
restatement of the same estimator (oracle/torch_ref.py) on the host cores,
with the C oracle's time beside it.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import subprocess
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

HBM_PEAK_GBPS = 8000.0  # MI355X published HBM3E bandwidth, 8 TB/s
METRIC = "sampled-attn decode µs/step + achieved HBM TB/s (B=8, 32k ctx, S=256); tokens/s"


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--warmup-ms", type=float, default=400.0,
                    help="minimum wall time of warm-up decode calls before timing")
    ap.add_argument("--windows", type=int, default=5,
                    help="alternating windows of the step and of the tile pass alone (medians reported)")
    ap.add_argument("--batch", type=int, default=8)
    ap.add_argument("--ctx", type=int, default=32768)
    ap.add_argument("--S", type=int, default=256)
    ap.add_argument("--seed", type=int, default=1690)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--workload", choices=("cfg2", "cfg3", "cfg4", "cfg5", "cfg5p", "single", "propgen",
                                           "flashragged"),
                    default="cfg2",
                    help="cfg2: the headline (flash, B=8, 32k); cfg3: batched ragged santa_prop (B=16, "
                         "L_b in [8192, 131072], S_b = L_b // 64); cfg4: model-level decode, random-init "
                         "Llama-3.1-8B shape, B=4, 32768-token prompt, 64 greedy steps, santa_flash S=256 vs exact; "
                         "cfg5: flash stress (B=32, 64q/8kv, 128k, S=512); cfg5p: santa_prop at cfg5's shape with "
                         "S=512 per sequence; single: one sequence of --ctx tokens through santa_flash (S=256) "
                         "and santa_prop (S=L/64); propgen: santa_prop on a shape outside the tuned kernels "
                         "(--heads/--kv-heads/--head-dim, default MHA 32q/32kv d=128), B=--batch, --ctx tokens, "
                         "S = L // 64 per sequence; flashragged: santa_flash on cfg3's lengths (B=16, "
                         "--heads query heads over 8 KV heads, one S = --S for the batch)")
    ap.add_argument("--heads", type=int, default=32, help="propgen: query heads")
    ap.add_argument("--kv-heads", type=int, default=32, help="propgen: KV heads")
    ap.add_argument("--head-dim", type=int, default=128, help="propgen: head_dim")
    ap.add_argument("--cpu-sample-seqs", type=int, default=8, help="sequences timed for the CPU baseline")
    ap.add_argument("--score-scale", type=float, default=1.0,
                    help="cfg4: multiply the query projections by this (every attention score that many times "
                         "larger); 1 is the random model's nearly uniform attention")
    ap.add_argument("--layers", type=int, default=0, help="cfg4: decoder layers (0: the 32 of Llama-3.1-8B)")
    ap.add_argument("--page-size", type=int, default=0,
                    help="cfg2 / cfg3 through the paged-KV entry point: the same tokens scattered over a pool of "
                         "pages of this many tokens in a seeded random order (0: contiguous cache)")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="first run a plain device copy of this many MiB 5 times (a known-size kernel "
                         "that calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    ap.add_argument("--extra-workloads", default="cfg3,cfg5,cfg5p,propgen,propgen_gqa7,propgen_gqa16,flashragged",
                    help="with the headline workload (cfg2, contiguous): after its own timing, also time these "
                         "workloads (20 steps each, 2 step windows) and report them under `extra_workloads` in the "
                         "same JSON line; '' for none")
    return ap.parse_args()


PMC_SUMMARY = os.path.join(REPO, "profiles", "flash_wave_kernel_cfg2_pmc.md")


def measured_traffic():
    """HBM bytes per launch of the tile kernel at the default workload, as
    recorded by the committed rocprofv3 --pmc summary (FETCH_SIZE +
    WRITE_SIZE, calibrated against a plain copy kernel); None if absent."""
    try:
        with open(PMC_SUMMARY) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(float(line.split(":", 1)[1].strip()))
    except OSError:
        pass
    return None


def make_inputs(B, L, H=32, KVH=8, D=128, seed=1690):
    import torch

    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, D, generator=g)
    K = torch.randn(B, L, KVH, D, generator=g)
    V = torch.randn(B, L, KVH, D, generator=g)
    C = torch.randn(B, L, KVH, 4, generator=g)
    U = torch.randn(KVH, 4, D, generator=g) / math.sqrt(D)
    K = K + 0.5 * math.sqrt(D) * torch.einsum("blkr,krd->blkd", C, U)
    return q.bfloat16(), K.bfloat16(), V.bfloat16()


def host_threads():
    """The host cores this process may use (the GPU box grants a share of the
    machine, which os.cpu_count() does not show)."""
    return int(os.environ.get("OMP_NUM_THREADS") or 0) or len(os.sched_getaffinity(0))


def cpu_model():
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(q, K, V, S, seed, n_seq, min_wall_s=2.0, min_steps=5, max_steps=20):
    """The reference algorithm's PyTorch CPU path (oracle/torch_ref.py, a
    vectorized restatement of the same estimator) on the host cores: whole
    decode steps of the first n_seq sequences, repeated for at least
    min_wall_s and min_steps, median step time.  Beside it, the C oracle
    (OpenMP over tiles) on the same sample."""
    import torch

    import oracle
    from oracle import torch_ref

    threads = host_threads()
    torch.set_num_threads(threads)
    qs, Ks, Vs = q[:n_seq].contiguous(), K[:n_seq].contiguous(), V[:n_seq].contiguous()

    def timed(fn, min_steps, max_steps, min_wall):
        fn()  # first call: allocations, thread pools
        times = []
        t_start = time.perf_counter()
        while len(times) < max_steps and (time.perf_counter() - t_start < min_wall or len(times) < min_steps):
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
        return statistics.median(times), len(times)

    dt, n = timed(lambda: torch_ref.flash_decode(qs, Ks, Vs, S, seed=seed), min_steps, max_steps, min_wall_s)
    dt_c, n_c = timed(lambda: oracle.flash_decode(qs, Ks, Vs, S, seed=seed, nthreads=threads), 3, 10, 1.0)
    return {"value": n_seq / dt, "unit": "tokens/s", "cores": threads, "kind": "port",
            "impl": "vectorized PyTorch CPU restatement (oracle/torch_ref.py)",
            "sample": f"{n_seq} of {q.shape[0]} sequences x 1 decode step (L={K.shape[1]}, S={S}); "
                      f"median of {n} steps, {dt:.3f} s each",
            "torch_num_threads": torch.get_num_threads(), "os_cpu_count": os.cpu_count(),
            "cpu_model": cpu_model(),
            "c_oracle": {"value": n_seq / dt_c, "unit": "tokens/s", "cores": threads,
                         "sample": f"same sample, median of {n_c} steps, {dt_c:.3f} s each; "
                                   "C restatement (oracle/santa_oracle.c), OpenMP over tiles"}}


def device_inputs(B, L, H, KVH, D, seed, dev, keys="bias"):
    """Synthetic q, K, V generated on the device (the larger workloads): N(0,1),
    with K either plus the rank-4 key bias of the headline recipe ("bias") or
    Student-t(3) with 16 planted needle rows per (b, kv) ("needles": K rows
    set to a multiple of the group's mean query direction, scoring ~6 nats
    above the rest)."""
    import torch

    g = torch.Generator(device=dev).manual_seed(seed)
    q = torch.randn(B, H, D, generator=g, device=dev)
    V = torch.randn(B, L, KVH, D, generator=g, device=dev, dtype=torch.bfloat16)
    if keys == "bias":
        K = torch.randn(B, L, KVH, D, generator=g, device=dev)
        C = torch.randn(B, L, KVH, 4, generator=g, device=dev)
        U = torch.randn(KVH, 4, D, generator=g, device=dev) / math.sqrt(D)
        K = (K + 0.5 * math.sqrt(D) * torch.einsum("blkr,krd->blkd", C, U)).bfloat16()
        del C
    else:
        K = torch.empty(B, L, KVH, D, device=dev, dtype=torch.bfloat16)
        for b in range(B):  # Student-t(3) = N / sqrt(chi2_3 / 3), one sequence at a time
            n = torch.randn(L, KVH, D, generator=g, device=dev)
            chi = (torch.randn(3, L, KVH, D, generator=g, device=dev) ** 2).sum(0) / 3.0
            K[b] = (n / chi.sqrt()).bfloat16()
        GH = H // KVH
        qm = q.view(B, KVH, GH, D).mean(2)
        qhat = qm / qm.norm(dim=-1, keepdim=True)
        alpha = (12.0 + 6.0) * math.sqrt(D) / qm.norm(dim=-1, keepdim=True)
        pos = torch.randint(0, L, (B, KVH, 16), generator=g, device=dev)
        for kv in range(KVH):
            K[torch.arange(B, device=dev)[:, None], pos[:, kv], kv] = (alpha[:, kv] * qhat[:, kv]).bfloat16()[:, None]
    return q.bfloat16(), K, V


def to_pages(K, V, P, seed):
    """K, V [B, L, KVH, D] on the device -> a pool [B * ceil(L / P), P, KVH, D]
    holding every sequence's pages in a seeded random order, and the int32
    block table [B, ceil(L / P)]."""
    import torch

    B, L, KVH, D = K.shape
    n = (L + P - 1) // P
    perm = torch.randperm(B * n, generator=torch.Generator().manual_seed(seed + 1)).to(K.device)
    pools = []
    for X in (K, V):
        if n * P != L:
            X = torch.cat([X, X.new_zeros(B, n * P - L, KVH, D)], dim=1)
        pool = torch.empty(B * n, P, KVH, D, dtype=X.dtype, device=X.device)
        pool[perm] = X.reshape(B * n, P, KVH, D)
        pools.append(pool)
    return pools[0], pools[1], perm.view(B, n).to(torch.int32).contiguous()


class Timing:
    """Warm-up by time, the official window of exactly `steps` calls, then
    alternating windows of the step and of the dominant kernel alone."""

    def __init__(self, args):
        self.args = args

    def _window(self, fn, n):
        import torch

        stream = torch.cuda.current_stream()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        # three untimed calls keep the GPU busy (and at its working clocks)
        # while the timed ones are submitted: e0 then fires when they end and
        # the window holds the n calls back to back, without the host's latency
        # to its first launch
        for _ in range(3):
            fn()
        e0.record(stream)
        for _ in range(n):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n, time.perf_counter() - t0

    def run(self, step, kernel=None):
        import torch

        a = self.args
        t0 = time.perf_counter()
        calls = 0
        for _ in range(a.warmup):
            step()
            calls += 1
        torch.cuda.synchronize()
        while time.perf_counter() - t0 < a.warmup_ms * 1e-3:
            for _ in range(20):
                step()
            calls += 20
            torch.cuda.synchronize()
        res = {"warmup_calls": calls, "warmup_s": time.perf_counter() - t0}
        # the official window: exactly `steps` calls
        res["ms_per_step"], res["wall_s_timed"] = self._window(step, a.steps)
        per = max(a.steps, 50)
        steps_w, kern_w = [], []
        for _ in range(max(1, a.windows)):
            steps_w.append(self._window(step, per)[0])
            if kernel is not None:
                kern_w.append(self._window(kernel, per)[0])
        res["step_windows_ms"] = steps_w
        res["ms_per_step_median"] = statistics.median(steps_w)
        if kernel is not None:
            res["kernel_windows_ms"] = kern_w
            res["kernel_ms"] = statistics.median(kern_w)
        res["window_calls"] = per
        return res


def base_line(metric, B, tm, args, dtype="bf16"):
    ms = tm["ms_per_step"]
    return {
        "metric": metric, "value": B / (ms * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "us_per_step": ms * 1e3,
        "us_per_step_median": tm["ms_per_step_median"] * 1e3, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": dtype, "data": "synthetic",
    }


def timing_keys(tm):
    return {"warmup_s": tm["warmup_s"], "warmup_calls": tm["warmup_calls"], "wall_s_timed": tm["wall_s_timed"],
            "windows": {"calls_each": tm["window_calls"],
                        "step_us": [round(x * 1e3, 2) for x in tm["step_windows_ms"]],
                        "kernel_us": [round(x * 1e3, 2) for x in tm.get("kernel_windows_ms", [])]}}


def roofline(bytes_alg, tm, kernel_name, traffic=None, v_rows=None):
    """Roofline block: achieved = algorithmic bytes / the dominant kernel's
    median duration (the whole step when there is no kernel timing)."""
    k_ms = tm.get("kernel_ms", tm["ms_per_step_median"])
    achieved = bytes_alg / (k_ms * 1e-3) / 1e9
    step_gbps = bytes_alg / (tm["ms_per_step"] * 1e-3) / 1e9
    r = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
         "frac": achieved / HBM_PEAK_GBPS, "traffic": traffic, "kernel": kernel_name, "kernel_us": k_ms * 1e3,
         "bytes_alg_per_launch": bytes_alg, "step_achieved_GBps": step_gbps, "step_frac": step_gbps / HBM_PEAK_GBPS,
         "kernel_le_step": k_ms <= tm["ms_per_step_median"]}
    if v_rows is not None:
        r["emitted_v_rows"] = v_rows
    return r


def flash_bytes(lens, KVH, H, B, v_rows, D=128):
    return sum(lens) * KVH * D * 2 + v_rows * D * 2 + B * H * D * 2 * 2 + B * H * 4


def run_cfg2(args, dev):
    import torch
    import santa_flash_batch_cuda as flash

    if args.copy_calibration_mib > 0:
        n = args.copy_calibration_mib << 20
        src = torch.ones(n // 2, dtype=torch.bfloat16, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    B, L, S, seed = args.batch, args.ctx, args.S, args.seed
    H, KVH, D = 32, 8, 128
    q_c, K_c, V_c = make_inputs(B, L, H, KVH, D, seed)
    q, K, V = q_c.to(dev), K_c.to(dev), V_c.to(dev)
    torch.cuda.synchronize()
    # untimed: emitted V rows for the algorithmic byte count
    _, _, vrows = flash.decode_systematic_batched(q, K, V, S, seed=seed, want_vrows=True)
    v_rows = int(vrows.sum().item())
    bytes_alg = flash_bytes([L] * B, KVH, H, B, v_rows)
    T_c = (L + 255) // 256
    ws = torch.empty(flash._workspace_bytes(B, H, KVH, D, T_c), dtype=torch.uint8, device=dev)

    def step():
        flash.decode_systematic_batched(q, K, V, S, seed=seed)

    def tiles():  # the step's dominant launch alone: the flash tile pass
        flash._decode_tiles_only(q, K, V, S, seed, 0, -1, ws)

    tm = Timing(args).run(step, tiles)
    default_workload = (B, L, S, seed) == (8, 32768, 256, 1690)
    line = base_line(METRIC, B, tm, args)
    line["config"] = {"workload": f"santa_flash decode, Llama-3.1-8B attention shape (32q/8kv, d=128), B={B}, "
                                  f"{L} cached tokens, S={S}, seed {seed}, K/V ~ N(0,1) + rank-4 key bias 0.5",
                      "global_batch": B, "seq_len": L, "S": S, "parallelism": "single GPU"}
    line["roofline"] = roofline(bytes_alg, tm, flash._tile_pass_kernel(B, H, KVH, T_c, 256),
                                measured_traffic() if default_workload else None, v_rows)
    line.update(timing_keys(tm))
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(q_c, K_c, V_c, S, seed, args.cpu_sample_seqs)
    return line


def run_cfg2_paged(args, dev):
    """The headline workload through decode_systematic_paged: the same tokens
    in a pool of args.page_size-token pages (seeded random page order)."""
    import torch
    import santa_flash_batch_cuda as flash

    B, L, S, seed, P = args.batch, args.ctx, args.S, args.seed, args.page_size
    H, KVH, D = 32, 8, 128
    q_c, K_c, V_c = make_inputs(B, L, H, KVH, D, seed)
    q = q_c.to(dev)
    Kp, Vp, table = to_pages(K_c.to(dev), V_c.to(dev), P, seed)
    torch.cuda.synchronize()
    lens = [L] * B

    def step(want_vrows=False):
        return flash.decode_systematic_paged(q, Kp, Vp, table, lens, S, seed=seed, want_vrows=want_vrows)

    _, _, vrows = step(True)
    v_rows = int(vrows.sum().item())
    tm = Timing(args).run(step)
    line = base_line(METRIC + " (paged KV)", B, tm, args)
    line["config"] = {"workload": f"santa_flash decode, Llama-3.1-8B attention shape (32q/8kv, d=128), B={B}, {L} "
                                  f"cached tokens in {P}-token pages (seeded random page order), S={S}, seed {seed}, "
                                  "K/V ~ N(0,1) + rank-4 key bias 0.5",
                      "global_batch": B, "seq_len": L, "S": S, "page_size": P, "parallelism": "single GPU"}
    line["roofline"] = roofline(flash_bytes(lens, KVH, H, B, v_rows), tm,
                                "whole paged decode step (tile pass + merge)", None, v_rows)
    line.update(timing_keys(tm))
    return line


def run_cfg3(args, dev):
    """Batched ragged santa_prop: B=16 sequences, L_b ~ U[8192, 131072] (seeded),
    S_b = L_b // 64, one decode_systematic_batched call per step."""
    import torch
    import santa_prop_batch_cuda as prop

    B, H, KVH, D, seed = 16, 32, 8, 128, args.seed
    gl = torch.Generator().manual_seed(seed)
    lens = torch.randint(8192, 131072 + 1, (B,), generator=gl).tolist()
    Ss = [l // 64 for l in lens]
    L = max(lens)
    q, K, V = device_inputs(B, L, H, KVH, D, seed, dev)
    torch.cuda.synchronize()
    P = args.page_size
    if P:
        Kp, Vp, table = to_pages(K, V, P, seed)
        del K, V

        def step(want_vrows=False):
            return prop.decode_systematic_paged(q, Kp, Vp, table, lens, Ss, seed=seed, want_vrows=want_vrows)
    else:
        def step(want_vrows=False):
            return prop.decode_systematic_batched(q, K, V, Ss, seed=seed, want_vrows=want_vrows, valid_len=lens)
    _, _, vrows = step(True)
    v_rows = int(vrows.sum().item())
    tm = Timing(args).run(step)
    line = base_line("sampled-attn decode µs/step + achieved HBM TB/s; tokens/s (cfg3: batched ragged santa_prop)",
                     B, tm, args)
    line["config"] = {"workload": f"santa_prop batched ragged decode, 32q/8kv, d=128, B={B}, L_b seeded U[8192, "
                                  f"131072] (sum {sum(lens)}), S_b = L_b // 64, seed {seed}, K/V ~ N(0,1) + rank-4 key "
                                  "bias 0.5" + (f", paged KV ({P}-token pages in a seeded random order)" if P else ""),
                      "global_batch": B, "seq_len": lens, "S": Ss, "parallelism": "single GPU"}
    line["roofline"] = roofline(flash_bytes(lens, KVH, H, B, v_rows), tm,
                                "whole prop step (pass 1 + budgets + pass 2 + finalize)", None, v_rows)
    line.update(timing_keys(tm))
    return line


def run_flashragged(args, dev):
    """Ragged santa_flash on cfg3's seeded lengths: B=16 sequences, L_b ~
    U[8192, 131072], one S for the batch (--S; S_per_tile from
    each sequence's tile count), --heads query heads over 8 KV heads, one
    decode_systematic_batched call per step."""
    import torch
    import santa_flash_batch_cuda as flash

    B, H, KVH, D, S, seed = 16, args.heads, 8, 128, args.S, args.seed
    gl = torch.Generator().manual_seed(seed)
    lens = torch.randint(8192, 131072 + 1, (B,), generator=gl).tolist()
    L = max(lens)
    q, K, V = device_inputs(B, L, H, KVH, D, seed, dev)
    torch.cuda.synchronize()

    def step(want_vrows=False):
        return flash.decode_systematic_batched(q, K, V, S, seed=seed, want_vrows=want_vrows, valid_len=lens)
    _, _, vrows = step(True)
    v_rows = int(vrows.sum().item())
    tm = Timing(args).run(step)
    line = base_line("sampled-attn decode µs/step + achieved HBM TB/s; tokens/s (ragged santa_flash on cfg3's "
                     "lengths)", B, tm, args)
    line["config"] = {"workload": f"santa_flash batched ragged decode, {H}q/{KVH}kv, d=128, B={B}, L_b seeded "
                                  f"U[8192, 131072] (sum {sum(lens)}), S={S}, seed {seed}, K/V ~ N(0,1) + rank-4 key "
                                  "bias 0.5", "global_batch": B, "seq_len": lens, "S": S, "parallelism": "single GPU"}
    line["roofline"] = roofline(flash_bytes(lens, KVH, H, B, v_rows), tm, "whole flash step (tile pass + merge)",
                                None, v_rows)
    line.update(timing_keys(tm))
    return line


def run_cfg5(args, dev):
    """Flash stress: B=32, 64q/8kv (GH 8), L=131072, S=512, Student-t(3) keys with
    planted needles."""
    import torch
    import santa_flash_batch_cuda as flash

    B, L, H, KVH, D, S, seed = 32, 131072, 64, 8, 128, 512, args.seed
    q, K, V = device_inputs(B, L, H, KVH, D, seed, dev, keys="needles")
    torch.cuda.synchronize()
    _, _, vrows = flash.decode_systematic_batched(q, K, V, S, seed=seed, want_vrows=True)
    v_rows = int(vrows.sum().item())
    T_c = (L + 255) // 256
    ws = torch.empty(flash._workspace_bytes(B, H, KVH, D, T_c), dtype=torch.uint8, device=dev)

    def step():
        flash.decode_systematic_batched(q, K, V, S, seed=seed)

    def tiles():
        flash._decode_tiles_only(q, K, V, S, seed, 0, -1, ws)

    tm = Timing(args).run(step, tiles)
    line = base_line("sampled-attn decode µs/step + achieved HBM TB/s; tokens/s (cfg5: flash stress)", B, tm, args)
    line["config"] = {"workload": f"santa_flash decode, 64q/8kv (GH 8), d=128, B={B}, {L} cached tokens, S={S}, "
                                  f"seed {seed}, Student-t(3) keys with 16 planted needles per KV head",
                      "global_batch": B, "seq_len": L, "S": S, "parallelism": "single GPU"}
    line["roofline"] = roofline(flash_bytes([L] * B, KVH, H, B, v_rows), tm,
                                flash._tile_pass_kernel(B, H, KVH, T_c, 256), None, v_rows)
    line.update(timing_keys(tm))
    return line


def run_cfg5p(args, dev):
    """santa_prop at cfg5's shape: B=32, 64q/8kv (GH 8: the general pass 1),
    L=131072, S=512 per sequence (the flash leg's budget), Student-t(3) keys
    with planted needles; one batched call per step."""
    import torch
    import santa_prop_batch_cuda as prop

    B, L, H, KVH, D, S, seed = 32, 131072, 64, 8, 128, 512, args.seed
    q, K, V = device_inputs(B, L, H, KVH, D, seed, dev, keys="needles")
    torch.cuda.synchronize()

    def step(want_vrows=False):
        return prop.decode_systematic_batched(q, K, V, S, seed=seed, want_vrows=want_vrows)

    _, _, vrows = step(True)
    v_rows = int(vrows.sum().item())
    tm = Timing(args).run(step)
    line = base_line("sampled-attn decode µs/step + achieved HBM TB/s; tokens/s (cfg5: santa_prop leg)", B, tm, args)
    line["config"] = {"workload": f"santa_prop batched decode, 64q/8kv (GH 8), d=128, B={B}, {L} cached tokens, "
                                  f"S={S} per sequence, seed {seed}, Student-t(3) keys with 16 planted needles per "
                                  "KV head",
                      "global_batch": B, "seq_len": L, "S": S, "parallelism": "single GPU"}
    line["roofline"] = roofline(flash_bytes([L] * B, KVH, H, B, v_rows), tm,
                                "whole prop step (pass 1 + budgets + pass 2 + finalize)", None, v_rows)
    line.update(timing_keys(tm))
    return line


def run_propgen(args, dev):
    """santa_prop on a shape the tuned pass-1 kernels do not take (default MHA
    32q/32kv, d=128; GQA 2/16 and head dims other than 128 likewise), B=--batch
    sequences of --ctx tokens, S = L // 64 per sequence, K/V ~ N(0,1); one
    batched call per step."""
    import torch
    import santa_prop_batch_cuda as prop

    B, L, H, KVH, D, seed = args.batch, args.ctx, args.heads, args.kv_heads, args.head_dim, args.seed
    S = max(1, L // 64)
    g = torch.Generator(device=dev).manual_seed(seed)
    q = torch.randn(B, H, D, device=dev, generator=g).bfloat16()
    K = torch.randn(B, L, KVH, D, device=dev, generator=g).bfloat16()
    V = torch.randn(B, L, KVH, D, device=dev, generator=g).bfloat16()
    torch.cuda.synchronize()

    def step(want_vrows=False):
        return prop.decode_systematic_batched(q, K, V, S, seed=seed, want_vrows=want_vrows)

    _, _, vrows = step(True)
    v_rows = int(vrows.sum().item())
    tm = Timing(args).run(step)
    line = base_line(f"sampled-attn decode µs/step + achieved HBM TB/s; tokens/s (santa_prop, {H}q/{KVH}kv, d={D})",
                     B, tm, args)
    line["config"] = {"workload": f"santa_prop batched decode, {H}q/{KVH}kv (GH {H // KVH}), d={D}, B={B}, {L} cached "
                                  f"tokens, S={S} per sequence, seed {seed}, K/V ~ N(0,1)",
                      "global_batch": B, "seq_len": L, "S": S, "parallelism": "single GPU"}
    line["roofline"] = roofline(flash_bytes([L] * B, KVH, H, B, v_rows, D=D), tm,
                                "whole prop step (pass 1 + budgets + pass 2 + finalize)", None, v_rows)
    line.update(timing_keys(tm))
    return line


def run_single(args, dev):
    """One sequence of --ctx tokens (32q/8kv, d=128, bf16, N(0,1) from the
    seeded device generator): santa_flash decode_systematic_batched at B=1
    (S=256) and santa_prop decode_systematic_scalar (S = L // 64), the
    short-call regime of a single request."""
    import torch
    import santa_flash_batch_cuda as flash
    import santa_prop_batch_cuda as prop

    L, H, KVH, D, seed = args.ctx, 32, 8, 128, args.seed
    g = torch.Generator(device=dev).manual_seed(seed)
    q = torch.randn(1, H, D, device=dev, generator=g).bfloat16()
    K = torch.randn(1, L, KVH, D, device=dev, generator=g).bfloat16()
    V = torch.randn(1, L, KVH, D, device=dev, generator=g).bfloat16()
    q1, K1, V1 = q[0].contiguous(), K[0].contiguous(), V[0].contiguous()
    S_f, S_p = 256, max(1, L // 64)
    _, _, vr = flash.decode_systematic_batched(q, K, V, S_f, seed=seed, want_vrows=True)
    _, _, vr_p = prop.decode_systematic_scalar(q1, K1, V1, S_p, seed=seed, want_vrows=True)
    v_rows, v_rows_p = int(vr.sum().item()), int(vr_p.sum().item())
    bn = 256 if L > 3072 else (64 if L > 1536 else 32)
    T_c = (L + bn - 1) // bn
    ws = torch.empty(flash._workspace_bytes(1, H, KVH, D, T_c), dtype=torch.uint8, device=dev)
    tm = Timing(args).run(lambda: flash.decode_systematic_batched(q, K, V, S_f, seed=seed),
                          lambda: flash._decode_tiles_only(q, K, V, S_f, seed, 0, -1, ws))
    tp = Timing(args).run(lambda: prop.decode_systematic_scalar(q1, K1, V1, S_p, seed=seed))
    line = base_line(f"sampled-attn decode µs/step + achieved HBM TB/s; tokens/s (single sequence, {L} tokens)",
                     1, tm, args)
    line["config"] = {"workload": f"one sequence, 32q/8kv, d=128, {L} cached tokens, N(0,1) keys and values, "
                                  f"seed {seed}: santa_flash S={S_f} (timed) and santa_prop S={S_p} (prop_leg)",
                      "global_batch": 1, "seq_len": L, "S": S_f, "parallelism": "single GPU"}
    line["roofline"] = roofline(flash_bytes([L], KVH, H, 1, v_rows), tm,
                                flash._tile_pass_kernel(1, H, KVH, T_c, bn), None, v_rows)
    line["prop_leg"] = {"us_per_step": tp["ms_per_step"] * 1e3, "us_per_step_median": tp["ms_per_step_median"] * 1e3,
                        "S": S_p, "roofline": roofline(flash_bytes([L], KVH, H, 1, v_rows_p), tp,
                                                       "whole prop step", None, v_rows_p)}
    line.update(timing_keys(tm))
    return line


def run_cfg4(args, dev):
    """Model-level decode: a random-init Llama-3.1-8B-shaped decoder (bf16,
    N(0, 0.02) weights), B=4 prompts of 32768 seeded random tokens, exact
    prefill into contiguous NHD caches, then 64 greedy tokens with santa_flash
    (S=256) as the attention of every layer, timed; the same 64 steps with
    exact float32 attention, teacher-forced on santa's tokens, give the
    per-step deviation of the logits."""
    import torch
    from santa_amd import attention_backends as ab
    from santa_amd.runtime import (LLAMA_3_1_8B, ExactDecodeBackend, NHDCache, RandomLlama, decode_deviation,
                                   greedy_decode)

    import dataclasses

    B, P, steps, S, seed = 4, 32768, 64, 256, args.seed
    shape = LLAMA_3_1_8B if args.layers <= 0 else dataclasses.replace(LLAMA_3_1_8B, layers=args.layers)
    model = RandomLlama(shape, seed=seed, device=dev, score_scale=args.score_scale)
    prompt = torch.randint(0, shape.vocab, (B, P), generator=torch.Generator().manual_seed(seed)).to(dev)
    cache = NHDCache(shape, B, P + steps, torch.bfloat16, dev)
    t0 = time.perf_counter()
    logits0 = model.prefill(prompt, cache)
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    cache_exact = cache.clone()
    flash = ab.SantaFlashBackend(S=S, seed=seed, block_n=None)
    greedy_decode(model, logits0, P, cache.clone(), flash, 3)  # warm-up (kernels, allocator)
    res = greedy_decode(model, logits0, P, cache, flash, steps)
    exact = greedy_decode(model, logits0, P, cache_exact, ExactDecodeBackend(), steps, forced=res["tokens"])
    dev_stats = decode_deviation(res["logits"], exact["logits"])
    tok_s = B * steps / res["decode_time_s"]
    n = len(dev_stats["max_abs"])
    # bytes of one decode step: every weight once, plus each layer's K rows
    # (all valid ones) and the sampled V rows are read by santa_flash
    params = sum(t.numel() for L in model.layers for t in L.values()) + 2 * model.embed.numel() + model.norm.numel()
    kv_bytes = shape.layers * B * (P + steps // 2) * shape.kv_heads * shape.head_dim * 2
    step_bytes = params * 2 + kv_bytes
    step_s = res["decode_time_s"] / max(1, res["decode_steps"])
    return {
        "metric": "sampled-attn decode µs/step + achieved HBM TB/s; tokens/s (cfg4: model-level decode)",
        "value": tok_s, "unit": "tokens/s", "n_gpus": 1, "steps": steps, "warmup": 3,
        "ms_per_step": step_s * 1e3, "us_per_step": step_s * 1e6, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"model-level greedy decode, random-init Llama-3.1-8B shape ({shape.layers} layers, "
                               f"4096 hidden, 32q/8kv, d=128, 14336 MLP, 128256 vocab; N(0, 0.02) bf16"
                               + (f", query projections x{args.score_scale:g}" if args.score_scale != 1.0 else "")
                               + f"), B={B}, {P}-token seeded random prompts, {steps} tokens, santa_flash S={S} in "
                               "every layer",
                   "global_batch": B, "seq_len": P, "S": S, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": step_bytes / step_s / 1e9, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": step_bytes / step_s / 1e9 / HBM_PEAK_GBPS, "traffic": None,
                     "kernel": "whole decode step (weights + every layer's K)", "bytes_per_step": step_bytes},
        "exact_fp32_tokens_per_s": B * steps / exact["decode_time_s"],
        "prefill_s": prefill_s,
        "deviation_vs_exact": {"steps": n, "max_abs_max": max(dev_stats["max_abs"]),
                               "mean_rel_mean": sum(dev_stats["mean_rel"]) / n,
                               "top1_agree_mean": sum(dev_stats["top1_agree"]) / n,
                               "logits_absmax": float(exact["logits"].abs().max().item())},
    }


def extra_workloads(args, dev):
    """The other BASELINE workloads (and the generic-shape one) timed after the
    headline in the same process, 20 steps each: a summary of each line."""
    import copy
    import torch

    runners = {"cfg3": run_cfg3, "cfg5": run_cfg5, "cfg5p": run_cfg5p, "propgen": run_propgen,
               "propgen_gqa7": run_propgen, "propgen_gqa16": run_propgen, "flashragged": run_flashragged}
    # santa_prop shapes outside the tuned kernels: MHA, Qwen2.5-7B's 28q/4kv
    # and Llama-3.1-405B's 128q/8kv (d = 128, B = 8, 32k tokens); santa_flash
    # on cfg3's ragged lengths at 32q/8kv with S = 512
    heads = {"propgen_gqa7": (28, 4), "propgen_gqa16": (128, 8), "flashragged": (32, 8)}
    out = []
    for name in [w.strip() for w in args.extra_workloads.split(",") if w.strip()]:
        sub = copy.copy(args)
        sub.steps, sub.warmup, sub.warmup_ms, sub.windows = 20, 2, 200.0, 2
        sub.no_cpu_baseline, sub.page_size, sub.copy_calibration_mib = True, 0, 0
        sub.batch, sub.ctx, sub.heads, sub.kv_heads, sub.head_dim = 8, 32768, 32, 32, 128
        sub.heads, sub.kv_heads = heads.get(name, (sub.heads, sub.kv_heads))
        if name == "flashragged":
            sub.S = 512
        print(f"[bench] extra workload {name}", file=sys.stderr, flush=True)
        try:
            if name not in runners:
                raise ValueError(f"unknown workload {name!r}")
            r = runners[name](sub, dev)
            rf = r["roofline"]
            e = {"name": name, "workload": r["config"]["workload"], "steps": sub.steps,
                 "us_per_step": r["us_per_step"], "us_per_step_median": r["us_per_step_median"],
                 "bytes_alg_per_launch": rf["bytes_alg_per_launch"], "step_frac": rf["step_frac"],
                 "emitted_v_rows": rf["emitted_v_rows"]}
            if rf.get("kernel_us") is not None and not rf["kernel"].startswith("whole"):
                e["kernel"], e["kernel_us"], e["kernel_frac"] = rf["kernel"], rf["kernel_us"], rf["frac"]
        except Exception as exc:  # report it, keep the headline line
            e = {"name": name, "error": f"{type(exc).__name__}: {exc}"}
        out.append(e)
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    return out


def main():
    args = parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU; multi-GPU runs are not part of it",
                          "n_gpus": args.gpus}))
        return 2
    import torch

    dev = torch.device("cuda:0")
    if args.workload == "cfg2":
        line = run_cfg2_paged(args, dev) if args.page_size else run_cfg2(args, dev)
        if not args.page_size and args.extra_workloads.strip():
            line["extra_workloads"] = extra_workloads(args, dev)
    else:
        line = {"cfg3": run_cfg3, "cfg4": run_cfg4, "cfg5": run_cfg5, "cfg5p": run_cfg5p,
                "single": run_single, "propgen": run_propgen, "flashragged": run_flashragged}[args.workload](args, dev)
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
