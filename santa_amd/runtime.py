"""Model-level decode around the sampled-attention path.

A Llama-architecture decoder (RMSNorm, rotary embeddings, grouped-query
attention, SwiGLU MLP) with seeded random weights, a contiguous NHD KV cache
per layer ([B, T_storage, KVH, D], the layout the santa kernels read), a
prefill that fills the caches, and a lockstep greedy decode loop that calls an
attention backend once per layer per step through the adapter contract
``backend.decode(q [B,H,D], k_nhd, v_nhd, valid_len) -> [B,H,D]``.

It plays the role of the reference's manual batched decode
(tutorial_code/runtime_common.py:501-571, generate_lockstep_batch :574-675,
alloc_nhd_caches_from_prefill :340-397) without its Hugging Face plumbing:
the weights are generated here (no checkpoint is loaded), the prefill writes
the NHD caches directly, and the greedy loop keeps the tokens on the device
(no host synchronisation per step).
"""
from __future__ import annotations

import ctypes
import math
import os
import time
from dataclasses import dataclass
from typing import Dict, List, Optional

import torch
import torch.nn.functional as F

__all__ = ["LlamaShape", "LLAMA_3_1_8B", "RandomLlama", "NHDCache", "ExactDecodeBackend", "causal_attention",
           "greedy_decode", "decode_deviation"]


@dataclass(frozen=True)
class LlamaShape:
    hidden: int
    intermediate: int
    heads: int
    kv_heads: int
    layers: int
    vocab: int
    rope_theta: float = 500000.0
    rms_eps: float = 1e-5

    @property
    def head_dim(self) -> int:
        return self.hidden // self.heads


# LlamaConfig(hidden_size=4096, intermediate_size=14336, num_attention_heads=32,
# num_key_value_heads=8, num_hidden_layers=32, rope_theta=5e5, vocab_size=128256)
LLAMA_3_1_8B = LlamaShape(hidden=4096, intermediate=14336, heads=32, kv_heads=8, layers=32, vocab=128256)


def _rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """LlamaRMSNorm's roundings (the reference's model, runtime_common.py:536):
    x·rsqrt(mean(x²) + eps) in float32, rounded to x's dtype, then times the
    weight in the weight's dtype."""
    xf = x.float()
    xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return w * xf.to(x.dtype)


class _FusedOps:
    """The library's fused decode-step kernels (santa_rt_* in santa_amd.h):
    residual add + RMSNorm, RoPE of q and k with the cache write, SwiGLU.
    Used for tensors on a GPU; the torch expressions above stay the CPU path
    and the prefill's.  A GPU decode step fails loudly if the library is not
    built."""

    _lib = None

    @classmethod
    def lib(cls):
        if cls._lib is None:
            path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libsanta_amd.so")
            if not os.path.exists(path):
                raise RuntimeError("santa_amd/libsanta_amd.so is not built (run __graft_entry__.build())")
            L = ctypes.CDLL(path)
            L.santa_last_error.restype = ctypes.c_char_p
            L.santa_rt_add_rms_norm.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int, ctypes.c_int, ctypes.c_float,
                                                                         ctypes.c_void_p]
            L.santa_rt_rope_write.argtypes = [ctypes.c_void_p] * 6 + [ctypes.c_int] * 4 + [
                ctypes.c_longlong, ctypes.c_int, ctypes.c_void_p]
            L.santa_rt_silu_mul.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                            ctypes.c_void_p]
            L.santa_rt_linear.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int] * 4 + [ctypes.c_void_p]
            L.santa_rt_linear_rope.argtypes = [ctypes.c_void_p] * 2 + [ctypes.c_int] * 2 + [ctypes.c_void_p] * 5 + [
                ctypes.c_int] * 3 + [ctypes.c_longlong, ctypes.c_int, ctypes.c_void_p]
            L.santa_rt_argmax.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
            cls._lib = L
        return cls._lib

    @classmethod
    def _check(cls, rc):
        if rc != 0:
            raise RuntimeError(cls.lib().santa_last_error().decode())

    @staticmethod
    def _stream(t: torch.Tensor):
        return torch.cuda.current_stream(t.device).cuda_stream

    @classmethod
    def add_rms_norm(cls, h: torch.Tensor, a: Optional[torch.Tensor], w: torch.Tensor, eps: float) -> torch.Tensor:
        """h += a (in place, bf16) when a is given; returns rms_norm(h) * w."""
        assert h.is_contiguous() and h.dtype == torch.bfloat16 and (a is None or a.is_contiguous())
        x = torch.empty_like(h)
        rows, hidden = h.numel() // h.shape[-1], h.shape[-1]
        cls._check(cls.lib().santa_rt_add_rms_norm(h.data_ptr(), a.data_ptr() if a is not None else None,
                                                   w.data_ptr(), x.data_ptr(), rows, hidden, eps, cls._stream(h)))
        return x

    @classmethod
    def rope_write(cls, qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, cache: "NHDCache", layer: int,
                   pos: int, heads: int, kv_heads: int, head_dim: int) -> torch.Tensor:
        """q rotated ([B, H, D]); k rotated and v written to the caches at pos."""
        assert qkv.is_contiguous() and cos.is_contiguous() and sin.is_contiguous()
        B = qkv.shape[0]
        q = torch.empty(B, heads, head_dim, dtype=qkv.dtype, device=qkv.device)
        kc, vc = cache.k[layer], cache.v[layer]
        cls._check(cls.lib().santa_rt_rope_write(qkv.data_ptr(), cos.data_ptr(), sin.data_ptr(), q.data_ptr(),
                                                 kc.data_ptr(), vc.data_ptr(), B, heads, kv_heads, head_dim,
                                                 kc.shape[1], pos, cls._stream(qkv)))
        return q

    @staticmethod
    def linear_fits(rows: int, K: int) -> bool:
        """Whether santa_rt_linear takes x [rows, K]: rows <= 8, K a multiple
        of 8, rows rounded up to 1, 2, 4 or 8 times K rounded up to 2048 at
        most 65536 (the x rows it stages in LDS)."""
        mp = 1 if rows <= 1 else 2 if rows <= 2 else 4 if rows <= 4 else 8
        return 1 <= rows <= 8 and K % 8 == 0 and mp * (-(-K // 2048) * 2048) <= 65536

    @classmethod
    def linear(cls, x: torch.Tensor, w: torch.Tensor, *, swiglu: bool = False) -> torch.Tensor:
        """bf16(x @ w.T) for few rows of x (santa_rt_linear; F.linear where
        the shape does not fit it).  swiglu: w holds the gate rows then the up
        rows, and the result is silu_mul of the product, in silu_mul's
        roundings."""
        rows, K = x.numel() // x.shape[-1], x.shape[-1]
        if not (cls.linear_fits(rows, K) and x.dtype == torch.bfloat16 and w.dtype == torch.bfloat16
                and x.is_contiguous() and w.is_contiguous() and x.data_ptr() % 16 == 0 and w.data_ptr() % 16 == 0):
            y = F.linear(x, w)
            return cls.silu_mul(y) if swiglu else y
        N = w.shape[0] // 2 if swiglu else w.shape[0]
        y = torch.empty(*x.shape[:-1], N, dtype=x.dtype, device=x.device)
        cls._check(cls.lib().santa_rt_linear(x.data_ptr(), w.data_ptr(), y.data_ptr(), rows, N, K, int(swiglu),
                                             cls._stream(x)))
        return y

    @classmethod
    def linear_rope(cls, x: torch.Tensor, w: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, cache: "NHDCache",
                    layer: int, pos: int, heads: int, kv_heads: int, head_dim: int) -> torch.Tensor:
        """rope_write(linear(x, w), ...) as one kernel (santa_rt_linear_rope):
        q rotated ([B, H, D]) returned, k rotated and v written to the caches
        at pos; the two calls where the shape does not fit it."""
        B, K = x.shape[0], x.shape[-1]
        if not (cls.linear_fits(B, K) and x.dtype == torch.bfloat16 and w.dtype == torch.bfloat16
                and x.is_contiguous() and w.is_contiguous() and x.data_ptr() % 16 == 0 and w.data_ptr() % 16 == 0
                and cos.is_contiguous() and sin.is_contiguous() and head_dim % 2 == 0):
            return cls.rope_write(cls.linear(x, w), cos, sin, cache, layer, pos, heads, kv_heads, head_dim)
        q = torch.empty(B, heads, head_dim, dtype=x.dtype, device=x.device)
        kc, vc = cache.k[layer], cache.v[layer]
        cls._check(cls.lib().santa_rt_linear_rope(x.data_ptr(), w.data_ptr(), B, K, cos.data_ptr(), sin.data_ptr(),
                                                  q.data_ptr(), kc.data_ptr(), vc.data_ptr(), heads, kv_heads,
                                                  head_dim, kc.shape[1], pos, cls._stream(x)))
        return q

    @classmethod
    def argmax(cls, logits: torch.Tensor) -> torch.Tensor:
        """torch.argmax(logits, dim=-1) for float32 rows (santa_rt_argmax)."""
        assert logits.dtype == torch.float32 and logits.is_contiguous()
        n = logits.shape[-1]
        rows = logits.numel() // n
        out = torch.empty(logits.shape[:-1], dtype=torch.int64, device=logits.device)
        cls._check(cls.lib().santa_rt_argmax(logits.data_ptr(), rows, n, out.data_ptr(), cls._stream(logits)))
        return out

    @classmethod
    def silu_mul(cls, gu: torch.Tensor) -> torch.Tensor:
        assert gu.is_contiguous()
        inter = gu.shape[-1] // 2
        rows = gu.numel() // gu.shape[-1]
        out = torch.empty(*gu.shape[:-1], inter, dtype=gu.dtype, device=gu.device)
        cls._check(cls.lib().santa_rt_silu_mul(gu.data_ptr(), out.data_ptr(), rows, inter, cls._stream(gu)))
        return out


def _rope_cos_sin(positions: torch.Tensor, head_dim: int, theta: float, dtype: torch.dtype):
    """cos/sin [..., head_dim] for integer positions (rotate-half convention)."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, device=positions.device, dtype=torch.float32) / head_dim))
    ang = positions.to(torch.float32)[..., None] * inv
    emb = torch.cat([ang, ang], dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def _rotate_half(x: torch.Tensor) -> torch.Tensor:
    h = x.shape[-1] // 2
    return torch.cat([-x[..., h:], x[..., :h]], dim=-1)


def _apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    return x * cos + _rotate_half(x) * sin


def causal_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, chunk: int = 512) -> torch.Tensor:
    """Exact causal GQA attention for a prefill: q [B, P, H, D], k/v
    [B, P, KVH, D] -> [B, P, H, D].  Query chunks of `chunk` positions; the
    products run on contiguous operands only (K is transposed once per call
    into a contiguous copy and every chunk is scored against all of it, the
    future positions masked), scores in the input dtype, softmax in float32."""
    B, P, H, D = q.shape
    KVH = k.shape[2]
    GH = H // KVH
    scale = 1.0 / math.sqrt(D)
    kt = k.permute(0, 2, 3, 1).reshape(B * KVH, D, P).contiguous()      # [B*KVH, D, P]
    vv = v.permute(0, 2, 1, 3).reshape(B * KVH, P, D).contiguous()      # [B*KVH, P, D]
    out = torch.empty(B, P, H, D, dtype=q.dtype, device=q.device)
    for c0 in range(0, P, chunk):
        c1 = min(P, c0 + chunk)
        C = c1 - c0
        # [B, C, KVH, GH, D] -> [B*KVH, GH*C, D]
        qc = q[:, c0:c1].reshape(B, C, KVH, GH, D).permute(0, 2, 3, 1, 4).reshape(B * KVH, GH * C, D).contiguous()
        sc = torch.bmm(qc, kt).float() * scale                                   # [B*KVH, GH*C, P]
        qpos = torch.arange(c0, c1, device=q.device).repeat(GH)                  # row r -> position
        mask = torch.arange(P, device=q.device)[None, :] > qpos[:, None]
        sc.masked_fill_(mask[None], float("-inf"))
        pr = torch.softmax(sc, dim=-1).to(q.dtype)
        del sc
        o = torch.bmm(pr, vv)                                                    # [B*KVH, GH*C, D]
        out[:, c0:c1] = o.view(B, KVH, GH, C, D).permute(0, 3, 1, 2, 4).reshape(B, C, H, D)
        del pr, o
    return out


class ExactDecodeBackend:
    """Exact dense decode attention in float32 with contiguous operands only
    (the comparator of the model-level decode; same adapter contract as the
    backends in santa_amd.attention_backends)."""

    name = "exact_fp32"
    exact_attention = True
    supports_true_batch_decode = True

    def decode(self, q_bhd: torch.Tensor, k_nhd: torch.Tensor, v_nhd: torch.Tensor, valid_len: int) -> torch.Tensor:
        B, H, D = q_bhd.shape
        KVH = k_nhd.shape[2]
        GH = H // KVH
        L = int(valid_len)
        k = k_nhd[:, :L].permute(0, 2, 1, 3).reshape(B * KVH, L, D).float().contiguous()    # [B*KVH, L, D]
        v = v_nhd[:, :L].permute(0, 2, 1, 3).reshape(B * KVH, L, D).float().contiguous()
        q = q_bhd.float().reshape(B * KVH, GH, D).transpose(1, 2).contiguous()              # [B*KVH, D, GH]
        sc = torch.bmm(k, q) * (1.0 / math.sqrt(D))                                          # [B*KVH, L, GH]
        p = torch.softmax(sc, dim=1).transpose(1, 2).contiguous()                            # [B*KVH, GH, L]
        o = torch.bmm(p, v)                                                                  # [B*KVH, GH, D]
        return o.reshape(B, H, D).to(q_bhd.dtype)

    def info(self) -> Dict[str, object]:
        return {"backend": self.name, "exact_attention": True, "supports_true_batch_decode": True}


class NHDCache:
    """Per-layer contiguous K/V caches [B, T_storage, KVH, D] (the santa layout)."""

    def __init__(self, shape: LlamaShape, batch: int, storage: int, dtype, device):
        D, KVH = shape.head_dim, shape.kv_heads
        self.k = [torch.zeros(batch, storage, KVH, D, dtype=dtype, device=device) for _ in range(shape.layers)]
        self.v = [torch.zeros(batch, storage, KVH, D, dtype=dtype, device=device) for _ in range(shape.layers)]
        self.storage = storage

    def clone(self) -> "NHDCache":
        c = object.__new__(NHDCache)
        c.k = [t.clone() for t in self.k]
        c.v = [t.clone() for t in self.v]
        c.storage = self.storage
        return c

    def write(self, layer: int, pos: int, k_bkd: torch.Tensor, v_bkd: torch.Tensor) -> None:
        """The step's K/V ([B, KVH, D]) into position pos (tutorial_code/runtime_common.py:551-554)."""
        self.k[layer][:, pos].copy_(k_bkd)
        self.v[layer][:, pos].copy_(v_bkd)


class RandomLlama:
    """A Llama-architecture decoder with seeded N(0, std) weights (RMSNorm
    weights 1).  QKV and gate/up projections are stored fused.

    score_scale multiplies the query projection, so every attention score is
    that many times larger: 1 keeps the random model's nearly uniform
    attention over a long context, larger values give the peaky attention of
    a trained model, the regime a sampled estimator is built for."""

    def __init__(self, shape: LlamaShape, *, seed: int = 1690, std: float = 0.02, dtype=torch.bfloat16,
                 device="cuda", score_scale: float = 1.0):
        self.shape = shape
        self.dtype = dtype
        self.device = torch.device(device)
        g = torch.Generator(device=self.device).manual_seed(seed)
        s = shape
        D = s.head_dim

        def w(*size):
            t = torch.empty(*size, dtype=dtype, device=self.device)
            t.normal_(0.0, std, generator=g)
            return t

        self.embed = w(s.vocab, s.hidden)
        self.lm_head = w(s.vocab, s.hidden)
        self.norm = torch.ones(s.hidden, dtype=dtype, device=self.device)
        self.layers: List[Dict[str, torch.Tensor]] = []
        for _ in range(s.layers):
            self.layers.append({
                "ln1": torch.ones(s.hidden, dtype=dtype, device=self.device),
                "ln2": torch.ones(s.hidden, dtype=dtype, device=self.device),
                "wqkv": w((s.heads + 2 * s.kv_heads) * D, s.hidden),
                "wo": w(s.hidden, s.heads * D),
                "wgu": w(2 * s.intermediate, s.hidden),
                "wd": w(s.hidden, s.intermediate),
            })
            if score_scale != 1.0:
                self.layers[-1]["wqkv"][:s.heads * D].mul_(score_scale)

    # ------------------------------------------------------------ pieces
    def _qkv(self, L: Dict[str, torch.Tensor], x: torch.Tensor):
        s, D = self.shape, self.shape.head_dim
        qkv = F.linear(x, L["wqkv"])
        q, k, v = qkv.split([s.heads * D, s.kv_heads * D, s.kv_heads * D], dim=-1)
        return q, k, v

    def _mlp(self, L: Dict[str, torch.Tensor], x: torch.Tensor) -> torch.Tensor:
        gu = F.linear(x, L["wgu"])
        gate, up = gu.chunk(2, dim=-1)
        return F.linear(F.silu(gate) * up, L["wd"])

    # ------------------------------------------------------------ prefill
    @torch.inference_mode()
    def prefill(self, tokens: torch.Tensor, cache: NHDCache, *, mlp_chunk: int = 8192,
                attn_chunk: int = 512) -> torch.Tensor:
        """Causal forward over the prompt tokens [B, P]; writes K/V of positions
        0..P-1 into the caches and returns the last position's logits [B, V]
        (float32).  Attention is exact (causal_attention)."""
        s, D = self.shape, self.shape.head_dim
        B, P = tokens.shape
        pos = torch.arange(P, device=self.device)
        cos, sin = _rope_cos_sin(pos, D, s.rope_theta, self.dtype)  # [P, D]
        h = self.embed[tokens]  # [B, P, hidden]
        for li, L in enumerate(self.layers):
            x = _rms_norm(h, L["ln1"], s.rms_eps)
            q, k, v = self._qkv(L, x)
            q = _apply_rope(q.view(B, P, s.heads, D), cos[:, None], sin[:, None])
            k = _apply_rope(k.view(B, P, s.kv_heads, D), cos[:, None], sin[:, None])
            v = v.view(B, P, s.kv_heads, D)
            cache.k[li][:, :P].copy_(k)
            cache.v[li][:, :P].copy_(v)
            a = causal_attention(q, k, v, chunk=attn_chunk)  # [B, P, H, D]
            del q, k, v, x
            h = h + F.linear(a.reshape(B, P, s.heads * D), L["wo"])
            del a
            for c0 in range(0, P, mlp_chunk):
                hc = h[:, c0:c0 + mlp_chunk]
                hc += self._mlp(L, _rms_norm(hc, L["ln2"], s.rms_eps))
        last = _rms_norm(h[:, -1], self.norm, s.rms_eps)
        return F.linear(last, self.lm_head).float()

    # ------------------------------------------------------------ decode
    @torch.inference_mode()
    def decode_step(self, token: torch.Tensor, pos: int, cache: NHDCache, backend) -> torch.Tensor:
        """One token per sequence (token [B]) at position pos: cache writes, the
        backend's attention over positions 0..pos, and the logits [B, V]
        (float32) -- tutorial_code/runtime_common.py:501-571."""
        s, D = self.shape, self.shape.head_dim
        B = token.shape[0]
        cos, sin = _rope_cos_sin(torch.tensor([pos], device=self.device), D, s.rope_theta, self.dtype)
        h = self.embed[token]  # [B, hidden]
        if self.device.type == "cuda" and self.dtype == torch.bfloat16:
            return self._decode_step_fused(h, cos.reshape(D).contiguous(), sin.reshape(D).contiguous(), pos, cache,
                                           backend)
        for li, L in enumerate(self.layers):
            x = _rms_norm(h, L["ln1"], s.rms_eps)
            q, k, v = self._qkv(L, x)
            q = _apply_rope(q.view(B, s.heads, D), cos, sin)
            k = _apply_rope(k.view(B, s.kv_heads, D), cos, sin)
            cache.write(li, pos, k, v.view(B, s.kv_heads, D))
            a = backend.decode(q.contiguous(), cache.k[li], cache.v[li], pos + 1)
            h = h + F.linear(a.reshape(B, s.heads * D), L["wo"])
            h = h + self._mlp(L, _rms_norm(h, L["ln2"], s.rms_eps))
        return F.linear(_rms_norm(h, self.norm, s.rms_eps), self.lm_head).float()

    def _decode_step_fused(self, h, cos, sin, pos, cache, backend):
        """decode_step on the GPU: per layer the four weight products as
        santa_rt_linear (the q/k/v product with RoPE and the cache write in its
        epilogue, the gate/up product with SwiGLU) and two fused add + norm
        kernels, around the backend's attention; the torch expressions'
        arithmetic and bf16 roundings, with each product accumulated in
        float32 in its own order."""
        s, D = self.shape, self.shape.head_dim
        B = h.shape[0]
        h = h.contiguous()
        x = _FusedOps.add_rms_norm(h, None, self.layers[0]["ln1"], s.rms_eps)
        lin = _FusedOps.linear
        for li, L in enumerate(self.layers):
            q = _FusedOps.linear_rope(x, L["wqkv"], cos, sin, cache, li, pos, s.heads, s.kv_heads, D)
            a = backend.decode(q, cache.k[li], cache.v[li], pos + 1)
            o = lin(a.reshape(B, s.heads * D), L["wo"])
            x = _FusedOps.add_rms_norm(h, o, L["ln2"], s.rms_eps)  # h += o
            m = lin(lin(x, L["wgu"], swiglu=True), L["wd"])
            nxt = self.layers[li + 1]["ln1"] if li + 1 < len(self.layers) else self.norm
            x = _FusedOps.add_rms_norm(h, m, nxt, s.rms_eps)  # h += m, then the next layer's (or final) norm
        return lin(x, self.lm_head).float()


@torch.inference_mode()
def greedy_decode(model: RandomLlama, first_logits: torch.Tensor, prompt_len: int, cache: NHDCache, backend,
                  steps: int, *, forced: Optional[torch.Tensor] = None) -> Dict[str, object]:
    """Lockstep greedy decode (tutorial_code/runtime_common.py:574-675):
    argmax of the current logits, one decode step per token, `steps` tokens
    per sequence.  With `forced` ([B, steps]) the given tokens are fed instead
    of the argmax (teacher forcing, for comparing backends on one trajectory).
    Returns the tokens [B, steps], the logits of every step [steps, B, V]
    and the decode time (events on the current stream)."""
    logits = first_logits
    toks, outs = [], []
    dev = first_logits.device
    timed = dev.type == "cuda"
    if timed:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
    t0 = time.perf_counter()
    pos = prompt_len
    for step in range(steps):
        if forced is not None:
            nxt = forced[:, step]
        elif timed and logits.dtype == torch.float32 and logits.is_contiguous():
            nxt = _FusedOps.argmax(logits)
        else:
            nxt = torch.argmax(logits, dim=-1)
        toks.append(nxt)
        outs.append(logits)
        if step == steps - 1:
            break
        logits = model.decode_step(nxt, pos, cache, backend)
        pos += 1
    if timed:
        e1.record()
        torch.cuda.synchronize()
        dt = e0.elapsed_time(e1) * 1e-3
    else:
        dt = time.perf_counter() - t0
    return {"tokens": torch.stack(toks, dim=1), "logits": torch.stack(outs, dim=0), "decode_time_s": dt,
            "decode_steps": steps - 1}


def decode_deviation(logits: torch.Tensor, ref: torch.Tensor) -> Dict[str, List[float]]:
    """Per-step max |a - b| and sum|a - b| / sum|b| of the logits [steps, B, V]."""
    err = (logits.float() - ref.float()).abs()
    max_abs = err.flatten(1).max(dim=1).values
    mean_rel = err.flatten(1).sum(dim=1) / ref.float().abs().flatten(1).sum(dim=1).clamp_min(1e-30)
    top1 = (logits.argmax(-1) == ref.argmax(-1)).float().mean(dim=1)
    return {"max_abs": max_abs.tolist(), "mean_rel": mean_rel.tolist(), "top1_agree": top1.tolist()}
