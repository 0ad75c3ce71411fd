"""CPU oracle for the S^2ANTA sampled-attention decode path.

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` -- never by the product package
``santa_amd`` or the extension modules.

The arithmetic lives in ``santa_oracle.c`` (a plain-C restatement of the
reference's kernels, compiled by ``oracle/Makefile``); this module is a thin
ctypes + numpy front end for it.  Tensors cross the boundary as raw 16-bit
patterns (``uint16``), so bf16 / f16 inputs are bit-identical to what the GPU
sees.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Dict, Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libsanta_oracle.so")
_lib: Optional[ctypes.CDLL] = None


def build(force: bool = False) -> str:
    """Compile the C restatement with ``make`` (gcc only)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE, "-B" if force else "all"], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        i32, u64, f32, i64 = ctypes.c_int, ctypes.c_uint64, ctypes.c_float, ctypes.c_long
        L.so_splitmix64.restype = u64
        L.so_splitmix64.argtypes = [u64]
        L.so_u01.restype = f32
        L.so_u01.argtypes = [u64, i32, i32]
        L.so_expf.restype = f32
        L.so_expf.argtypes = [f32]
        L.so_expf_array.restype = None
        L.so_expf_array.argtypes = [P, P, i64]
        L.so_u01_array.restype = None
        L.so_u01_array.argtypes = [u64, P, P, P, i64]
        L.so_counts_1d.restype = None
        L.so_counts_1d.argtypes = [P, i32, f32, f32, i32, P]
        L.so_auto_block_n.restype = i32
        L.so_auto_block_n.argtypes = [i32]
        L.so_flash_s_per_tile.restype = i32
        L.so_flash_s_per_tile.argtypes = [ctypes.c_int64, i32]
        L.so_bf16_to_f32.restype = f32
        L.so_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.so_f32_to_bf16.restype = ctypes.c_uint16
        L.so_f32_to_bf16.argtypes = [f32]
        L.so_f16_to_f32.restype = f32
        L.so_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.so_f32_to_f16.restype = ctypes.c_uint16
        L.so_f32_to_f16.argtypes = [f32]
        L.so_flash_decode.restype = i32
        L.so_flash_decode.argtypes = [P, P, P, i32, i32, i32, i32, i32, i32, i32, i32, u64,
                                      P, P, P, P, P, P, P, P, i32]
        L.so_flash_decode_at.restype = i32
        L.so_flash_decode_at.argtypes = [P, P, P, i32, i32, i32, i32, i32, i32, i32, i32, u64,
                                         P, P, P, P, P, P, P, P, i32, i32]
        L.so_f32_to_h16_array.restype = None
        L.so_f32_to_h16_array.argtypes = [P, P, i64, i32]
        L.so_h16_to_f32_array.restype = None
        L.so_h16_to_f32_array.argtypes = [P, P, i64, i32]
        L.so_prop_budgets.restype = None
        L.so_prop_budgets.argtypes = [P, P, i32, i32, u64, i32, P, P, P, P]
        L.so_prop_decode.restype = i32
        L.so_prop_decode.argtypes = [P, P, P, i32, i32, i32, i32, i32, i32, u64, i32,
                                     P, P, P, P, P, P, P, P, P, P, P]
        L.so_prop_decode_d.restype = i32
        L.so_prop_decode_d.argtypes = [P, P, P, i32, i32, i32, i32, i32, i32, i32, u64, i32,
                                       P, P, P, P, P, P, P, P, P, P, P]
        _lib = L
    return _lib


def _ptr(a: Optional[np.ndarray]):
    return None if a is None else ctypes.c_void_p(a.ctypes.data)


def as_bits(x) -> np.ndarray:
    """bf16/f16 torch tensor (any device) or uint16/int16 numpy array -> contiguous uint16 bits."""
    if isinstance(x, np.ndarray):
        return np.ascontiguousarray(x.view(np.uint16) if x.dtype == np.int16 else x.astype(np.uint16, copy=False))
    import torch

    t = x.detach().to("cpu").contiguous()
    if t.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError(f"expected bf16/f16 tensor, got {t.dtype}")
    return t.view(torch.int16).numpy().view(np.uint16).copy()


# ---------------------------------------------------------------- scalars
def splitmix64(x: int) -> int:
    return int(lib().so_splitmix64(ctypes.c_uint64(x & 0xFFFFFFFFFFFFFFFF)))


def u01(seed: int, key: int, t: int) -> float:
    return float(lib().so_u01(seed & 0xFFFFFFFFFFFFFFFF, key, t))


def expf(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().so_expf_array(_ptr(x), _ptr(y), x.size)
    return y


def f32_to_h16(x: np.ndarray, is_bf16: bool = True) -> np.ndarray:
    """f32 -> bf16 / f16 bits, round to nearest even (the kernels' conversion)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.uint16)
    lib().so_f32_to_h16_array(_ptr(x), _ptr(y), x.size, int(is_bf16))
    return y


def h16_to_f32(bits: np.ndarray, is_bf16: bool = True) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    y = np.empty(b.shape, dtype=np.float32)
    lib().so_h16_to_f32_array(_ptr(b), _ptr(y), b.size, int(is_bf16))
    return y


def u01_array(seed: int, key: np.ndarray, t: np.ndarray) -> np.ndarray:
    key = np.ascontiguousarray(key, dtype=np.int32)
    t = np.ascontiguousarray(t, dtype=np.int32)
    out = np.empty(key.shape, dtype=np.float32)
    lib().so_u01_array(seed & 0xFFFFFFFFFFFFFFFF, _ptr(key), _ptr(t), _ptr(out), key.size)
    return out


def counts_1d(ub_bits: np.ndarray, invdel: float, a0: float, is_bf16: bool = True) -> np.ndarray:
    ub = np.ascontiguousarray(ub_bits, dtype=np.uint16)
    c = np.zeros(ub.size, dtype=np.int16)
    lib().so_counts_1d(_ptr(ub), ub.size, invdel, a0, int(is_bf16), _ptr(c))
    return c


def auto_block_n(L: int) -> int:
    return int(lib().so_auto_block_n(L))


def flash_s_per_tile(S: int, T_c: int) -> int:
    return int(lib().so_flash_s_per_tile(S, T_c))


# ---------------------------------------------------------------- flash
def flash_decode(q, K, V, S: int, seed: int = 42, block_n: int = 0, valid_len: int = -1,
                 is_bf16: bool = True, debug: bool = False, nthreads: int = 0,
                 b_offset: int = 0) -> Dict[str, np.ndarray]:
    """Oracle of santa_flash_batch_cuda.decode_systematic_batched.

    q [B,H,128] or [H,128]; K,V [B,L,KVH,128] or [L,KVH,128] as bf16/f16
    tensors or uint16 bit arrays.  Returns a dict with ``out16`` (bits),
    ``out`` (f32 before the cast), ``m_star`` and, with ``debug``, the tile
    statistics ``m_tiles``, ``ell_tiles``, ``counts`` [B,H,T_c,BN],
    ``out_tiles`` and ``rowmask``.  ``b_offset``: these B sequences are
    sequences b_offset .. b_offset+B-1 of a batch (RNG key (b + b_offset)*H + h),
    e.g. one sequence of a ragged batch decoded on its own length."""
    qb, Kb, Vb = as_bits(q), as_bits(K), as_bits(V)
    single = qb.ndim == 2
    if single:
        qb, Kb, Vb = qb[None], Kb[None], Vb[None]
    B, H, D = qb.shape
    L_st, KVH = Kb.shape[1], Kb.shape[2]
    assert D == 128
    L = valid_len if valid_len > 0 else L_st
    bn = block_n if block_n > 0 else auto_block_n(L)
    T_c = (L + bn - 1) // bn
    S_pt = flash_s_per_tile(S, T_c)
    res = {
        "out": np.zeros((B, H, D), np.float32),
        "out16": np.zeros((B, H, D), np.uint16),
        "m_star": np.zeros((B, H), np.float32),
        "block_n": bn, "T_c": T_c, "S_per_tile": S_pt,
    }
    if debug:
        res["m_tiles"] = np.zeros((B, H, T_c), np.float32)
        res["ell_tiles"] = np.zeros((B, H, T_c), np.float32)
        res["counts"] = np.zeros((B, H, T_c, bn), np.int16)
        res["out_tiles"] = np.zeros((B, H, T_c, D), np.float32)
        res["rowmask"] = np.zeros((B, KVH, L), np.int32)
    rc = lib().so_flash_decode_at(
        _ptr(qb), _ptr(Kb), _ptr(Vb), int(is_bf16), B, H, KVH, L, L_st, bn, S_pt, seed & 0xFFFFFFFFFFFFFFFF,
        _ptr(res["out"]), _ptr(res["out16"]), _ptr(res["m_star"]), _ptr(res.get("m_tiles")),
        _ptr(res.get("ell_tiles")), _ptr(res.get("counts")), _ptr(res.get("out_tiles")),
        _ptr(res.get("rowmask")), int(nthreads), int(b_offset))
    if rc != 0:
        raise RuntimeError(f"so_flash_decode failed: {rc}")
    if debug:
        res["vrows"] = res["rowmask"].sum(axis=2).astype(np.int32)
    if single:
        for k in ("out", "out16", "m_star", "m_tiles", "ell_tiles", "counts", "out_tiles", "rowmask", "vrows"):
            if k in res:
                res[k] = res[k][0]
    return res


# ---------------------------------------------------------------- prop
def prop_budgets(m_tiles: np.ndarray, ell_tiles: np.ndarray, S: int, seed: int, h: int):
    m = np.ascontiguousarray(m_tiles, np.float32)
    e = np.ascontiguousarray(ell_tiles, np.float32)
    T_c = m.size
    ms = np.zeros(1, np.float32)
    St = np.zeros(T_c, np.int32)
    inv = np.zeros(T_c, np.float32)
    a0 = np.zeros(T_c, np.float32)
    lib().so_prop_budgets(_ptr(m), _ptr(e), T_c, int(S), seed & 0xFFFFFFFFFFFFFFFF, h, _ptr(ms), _ptr(St),
                          _ptr(inv), _ptr(a0))
    return {"m_star": float(ms[0]), "S_tiles": St, "invdelta": inv, "a0": a0}


def prop_pass1_mode(GH: int, D: int, bn: int, env: Optional[str] = None) -> int:
    """0 = vec path, 1 = general (MMA) path; prop/santa_cuda.cpp:39-51,212-229."""
    mode = (env or "").strip().lower()
    can_vec = GH == 4 and D == 128 and bn == 256
    if mode in ("vec", "gqa_vec"):
        return 0
    if mode in ("gqa", "perhead"):
        return 1
    return 0 if can_vec else 1


def prop_decode(q, K, V, S: int, seed: int = 42, block_n: int = 0, is_bf16: bool = True,
                pass1_mode: Optional[int] = None, debug: bool = False) -> Dict[str, np.ndarray]:
    """Oracle of santa_prop_batch_cuda.decode_systematic_scalar for one sequence:
    q [H,D]; K,V [L,KVH,D] (D a multiple of 16 up to 1024; block_n a multiple
    of 16 up to 512)."""
    qb, Kb, Vb = as_bits(q), as_bits(K), as_bits(V)
    H, D = qb.shape
    L, KVH = Kb.shape[0], Kb.shape[1]
    GH = H // KVH
    bn = block_n if block_n > 0 else (256 if (os.environ.get("SANTA_PASS1", "").lower() in ("vec", "gqa_vec"))
                                       else auto_block_n(L))
    T_c = (L + bn - 1) // bn
    mode = prop_pass1_mode(GH, D, bn, os.environ.get("SANTA_PASS1")) if pass1_mode is None else pass1_mode
    res = {
        "out": np.zeros((H, D), np.float32),
        "out16": np.zeros((H, D), np.uint16),
        "m_star": np.zeros(H, np.float32),
        "block_n": bn, "T_c": T_c, "pass1_mode": mode,
    }
    if debug:
        for k, dt in (("m_tiles", np.float32), ("ell_tiles", np.float32), ("S_tiles", np.int32),
                      ("invdelta", np.float32), ("a0", np.float32)):
            res[k] = np.zeros((H, T_c), dt)
        res["u_stash"] = np.zeros((L, H), np.uint16)
        res["counts"] = np.zeros((H, T_c, bn), np.int16)
        res["rowmask"] = np.zeros((KVH, L), np.int32)
    rc = lib().so_prop_decode_d(
        _ptr(qb), _ptr(Kb), _ptr(Vb), int(is_bf16), H, KVH, D, L, bn, int(S), seed & 0xFFFFFFFFFFFFFFFF, mode,
        _ptr(res["out"]), _ptr(res["out16"]), _ptr(res["m_star"]), _ptr(res.get("m_tiles")),
        _ptr(res.get("ell_tiles")), _ptr(res.get("S_tiles")), _ptr(res.get("invdelta")), _ptr(res.get("a0")),
        _ptr(res.get("u_stash")), _ptr(res.get("counts")), _ptr(res.get("rowmask")))
    if rc != 0:
        raise RuntimeError(f"so_prop_decode failed: {rc}")
    if debug:
        res["vrows"] = res["rowmask"].sum(axis=1).astype(np.int32)
    return res
