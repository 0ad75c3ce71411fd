"""Writes the golden fixtures of the santa_flash / santa_prop decode path.

    python tests/golden/make_golden.py

The fixtures are outputs of this repository's CPU oracle (oracle/, a C
restatement of the reference algorithm pinned by tests/test_oracle.py) on
inputs from tests/helpers.gen_qkv -- a seeded torch CPU generator, so the
inputs are not stored, only their SHA-256 digest (checked before use).  The
reference holds no test vectors of its own for this path.

Each .npz holds plain arrays (no pickles):
  digest            sha256 prefix of the q, K, V bit patterns
  spec              the gen_qkv / decode arguments, as a JSON string
  m_star, m_tiles, ell_tiles    f32 bit patterns (uint32)
  samples           int32 [n, 4]: (b*H + h, t, row, count) of every nonzero count
  out16             the 16-bit output bits
  S_tiles           (prop only) the per-tile budgets
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)
sys.path.insert(0, os.path.dirname(HERE))

CASES = {
    # batch 1, 32q/8kv, d=128, L=4096, S=32, seed 1690
    "flash_cfg1": dict(kind="flash", B=1, H=32, KVH=8, L=4096, gen_seed=1690, lowrank=0.0, S=32, seed=1690,
                       block_n=0, valid_len=-1),
    # ragged, auto block_n 64, valid_len below storage, GH 8
    "flash_gh8_ragged": dict(kind="flash", B=2, H=64, KVH=8, L=2600, gen_seed=1691, lowrank=0.5, S=200, seed=7,
                             block_n=0, valid_len=2345),
    # prop, vec path: L=5000, S = L // 64
    "prop_vec": dict(kind="prop", B=1, H=32, KVH=8, L=5000, gen_seed=1692, lowrank=0.5, S=78, seed=1690, block_n=0),
    # prop, general path (BN 64)
    "prop_general": dict(kind="prop", B=1, H=32, KVH=8, L=2000, gen_seed=1693, lowrank=0.0, S=64, seed=1690,
                         block_n=0),
}


def inputs(spec):
    from helpers import gen_qkv

    return gen_qkv(spec["B"], spec["H"], spec["KVH"], spec["L"], seed=spec["gen_seed"], lowrank=spec["lowrank"],
                   single=spec["kind"] == "prop")


def compute(spec):
    import oracle
    from helpers import tensor_digest

    q, K, V = inputs(spec)
    if spec["kind"] == "flash":
        r = oracle.flash_decode(q, K, V, spec["S"], seed=spec["seed"], block_n=spec["block_n"],
                                valid_len=spec["valid_len"], debug=True)
        c = r["counts"]  # [B,H,T_c,BN]
        B, H, T_c, BN = c.shape
        c = c.reshape(B * H, T_c, BN)
    else:
        r = oracle.prop_decode(q, K, V, spec["S"], seed=spec["seed"], block_n=spec["block_n"], debug=True)
        c = r["counts"]  # [H,T_c,BN]
    nz = np.argwhere(c > 0)
    samples = np.concatenate([nz, c[tuple(nz.T)][:, None]], axis=1).astype(np.int32)
    out = {
        "digest": np.array(tensor_digest(q, K, V)),
        "spec": np.array(json.dumps(spec, sort_keys=True)),
        "m_star": np.ascontiguousarray(r["m_star"]).view(np.uint32),
        "m_tiles": np.ascontiguousarray(r["m_tiles"]).view(np.uint32),
        "ell_tiles": np.ascontiguousarray(r["ell_tiles"]).view(np.uint32),
        "samples": samples,
        "out16": r["out16"],
    }
    if spec["kind"] == "prop":
        out["S_tiles"] = r["S_tiles"]
    return out


def main():
    for name, spec in CASES.items():
        out = compute(spec)
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **out)
        print(f"{path}: {len(out['samples'])} sampled (head, tile, row) entries")


if __name__ == "__main__":
    main()
