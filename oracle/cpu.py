"""TEST INFRASTRUCTURE — CPU oracle functions (numpy + the C restatement).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this
module.  bf16 tensors travel as numpy uint16 arrays holding the raw bits.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

_LIB_PATH = Path(__file__).resolve().parent / "liboracle_fd.so"
_LIB = None


def _lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not _LIB_PATH.exists():
            from . import build as _build
            _build.build()
        lib = ctypes.CDLL(str(_LIB_PATH))
        p = ctypes.c_void_p
        lib.fd_oracle_conv_taps.restype = None
        lib.fd_oracle_conv_taps.argtypes = [p, p, p, p, ctypes.c_int64, ctypes.c_int]
        lib.fd_oracle_silu.restype = ctypes.c_float
        lib.fd_oracle_silu.argtypes = [ctypes.c_float]
        lib.fd_oracle_f32_to_bf16.restype = ctypes.c_uint16
        lib.fd_oracle_f32_to_bf16.argtypes = [ctypes.c_float]
        lib.fd_oracle_packed_conv.restype = ctypes.c_int
        lib.fd_oracle_packed_conv.argtypes = [p, p, p, p, p, p] + [ctypes.c_int] * 5 + [p, ctypes.c_int, ctypes.c_int]
        lib.fd_oracle_attn_prologue.restype = ctypes.c_int
        lib.fd_oracle_attn_prologue.argtypes = [p, ctypes.c_int64, ctypes.c_int, p, ctypes.c_int, ctypes.c_int,
                                                ctypes.c_float, p, p, ctypes.c_int, p]
        lib.fd_oracle_add_rmsnorm.restype = ctypes.c_int
        lib.fd_oracle_add_rmsnorm.argtypes = [p, p, p, p, p, ctypes.c_int64, ctypes.c_int, ctypes.c_float,
                                              ctypes.c_int, ctypes.c_int]
        _LIB = lib
    return _LIB


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


# ------------------------------------------------------------------ bf16 bits

def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bits; NaN -> 0x7fc0 (torch's rule)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = 0x7FC0
    return r


def silu(y: float) -> float:
    """The conv's fp32 SiLU, y / (1 + expf(-y)) with the C library's expf."""
    return _lib().fd_oracle_silu(float(y))


# ------------------------------------------------------------- packed conv

def packed_conv(x_bits: np.ndarray, w_bits: np.ndarray, bias_bits: np.ndarray | None = None, *,
                key_dim: int | None = None, value_dim: int | None = None,
                cu_seqlens: np.ndarray | None = None, activation: str | None = "silu"):
    """Packed causal depthwise conv1d (+ SiLU) with q/k/v split.

    Restates ref: src/decider/packed_conv_kernel.py:128-191.  x_bits [B, T, C],
    w_bits [C, W] (or [C, 1, W]); returns (q, k, v) bits [B, T, key_dim] /
    [B, T, value_dim].
    """
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16)
    B, T, C = x_bits.shape
    w = np.ascontiguousarray(np.asarray(w_bits, dtype=np.uint16).reshape(C, -1))
    width = w.shape[1]
    if key_dim is None:
        key_dim = value_dim = C // 3
    assert C == 2 * key_dim + value_dim
    bias = None if bias_bits is None else np.ascontiguousarray(bias_bits, dtype=np.uint16)
    cu = None
    n_seqs = 0
    if cu_seqlens is not None:
        cu = np.ascontiguousarray(cu_seqlens, dtype=np.int32)
        n_seqs = cu.size - 1
    q = np.empty((B, T, key_dim), np.uint16)
    k = np.empty((B, T, key_dim), np.uint16)
    v = np.empty((B, T, value_dim), np.uint16)
    rc = _lib().fd_oracle_packed_conv(_ptr(x_bits), _ptr(w), _ptr(bias), _ptr(q), _ptr(k), _ptr(v), B, T,
                                      key_dim, value_dim, width, _ptr(cu), n_seqs,
                                      1 if activation == "silu" else 0)
    if rc != 0:
        raise ValueError("oracle packed_conv rejected its arguments")
    return q, k, v


def conv_taps(x_windows: np.ndarray, w_bits: np.ndarray, bias_bits: np.ndarray | None = None) -> np.ndarray:
    """fp32 pre-activation of independent conv outputs: x_windows [n, W] (oldest row first)
    and w_bits [n, W] bf16 bits, bias_bits [n] or None.  The same arithmetic as packed_conv."""
    xw = np.ascontiguousarray(x_windows, dtype=np.uint16)
    w = np.ascontiguousarray(w_bits, dtype=np.uint16)
    n, width = xw.shape
    assert w.shape == (n, width) and 1 <= width <= 4
    bias = None if bias_bits is None else np.ascontiguousarray(bias_bits, dtype=np.uint16)
    out = np.empty(n, np.float32)
    _lib().fd_oracle_conv_taps(_ptr(xw), _ptr(w), _ptr(bias), _ptr(out), n, width)
    return out


def packed_conv_f64(x_bits: np.ndarray, w_bits: np.ndarray, bias_bits=None, *, key_dim=None, value_dim=None,
                    activation: str | None = "silu") -> np.ndarray:
    """fp64 tap loop of the same conv, one final bf16 rounding: the reference's own test
    oracle (ref: experiments/packed_conv/check_packed_output_conv.py:21-32), generalised.
    Returns bf16 bits [B, T, C] before the q/k/v split."""
    x = bf16_to_f32(x_bits).astype(np.float64)
    B, T, C = x.shape
    w = bf16_to_f32(np.asarray(w_bits).reshape(C, -1)).astype(np.float64)
    width = w.shape[1]
    acc = np.zeros_like(x)
    for tap in range(width):
        lag = width - 1 - tap
        acc[:, lag:, :] += x[:, :T - lag, :] * w[:, tap]
    if bias_bits is not None:
        acc += bf16_to_f32(bias_bits).astype(np.float64)
    if activation == "silu":
        acc = acc / (1.0 + np.exp(-acc))
    return _f64_to_bf16(acc)


def _f64_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round fp64 straight to bf16 (nearest even) without an fp32 step."""
    x = np.asarray(x, dtype=np.float64)
    out = np.empty(x.shape, np.uint16)
    flat = x.reshape(-1)
    o = out.reshape(-1)
    f32 = flat.astype(np.float32)  # candidate neighbours: truncate the fp32 image, then fix up exactly
    bits = f32.view(np.uint32)
    lo = (bits >> 16).astype(np.uint32)
    cand_lo = (lo << 16).view(np.float32).astype(np.float64)
    # next bf16 away from zero in magnitude
    hi = lo + 1
    cand_hi = (hi.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    d_lo = np.abs(flat - cand_lo)
    d_hi = np.abs(flat - cand_hi)
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & ((lo & 1) == 1))
    res = np.where(pick_hi, hi, lo).astype(np.uint16)
    res[np.isnan(flat)] = 0x7FC0
    o[:] = res
    return out


# ------------------------------------------------------------- add + RMSNorm

def add_rmsnorm(x_bits: np.ndarray, residual_bits: np.ndarray | None, weight, eps: float = 1e-6,
                gain_offset: bool = True):
    """Fused residual add + RMSNorm (fp32 sequence of the kernel; see fd_oracle.c).

    weight: bf16 bits (uint16) or float32 array [width].  Returns (out_bits,
    residual_out_bits or None).
    """
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    width = x.shape[-1]
    rows = x.size // width
    res = None if residual_bits is None else np.ascontiguousarray(residual_bits, dtype=np.uint16)
    w = np.ascontiguousarray(weight)
    if w.dtype == np.uint16:
        wdt = 0
    else:
        w = w.astype(np.float32)
        wdt = 1
    out = np.empty_like(x)
    res_out = None if res is None else np.empty_like(x)
    rc = _lib().fd_oracle_add_rmsnorm(_ptr(x), _ptr(res), _ptr(w), _ptr(out), _ptr(res_out), rows, width,
                                      float(eps), wdt, 1 if gain_offset else 0)
    if rc != 0:
        raise ValueError("oracle add_rmsnorm rejected its arguments")
    return out, res_out


def add_rmsnorm_f64(x_bits, residual_bits, weight, eps: float = 1e-6, gain_offset: bool = True) -> np.ndarray:
    """Exact-arithmetic form: h = bf16(x + r) (fp32 add, as eager), then
    h * (mean(h^2) + eps)^-1/2 * g in fp64, one rounding to bf16."""
    x = bf16_to_f32(x_bits)
    if residual_bits is not None:
        h = bf16_to_f32(f32_to_bf16(x + bf16_to_f32(residual_bits))).astype(np.float64)
    else:
        h = x.astype(np.float64)
    w = np.asarray(weight)
    g = (bf16_to_f32(w) if w.dtype == np.uint16 else w.astype(np.float32)).astype(np.float64)
    if gain_offset:
        g = 1.0 + g
    ms = np.mean(h * h, axis=-1, keepdims=True)
    return _f64_to_bf16(h / np.sqrt(ms + eps) * g)


# ------------------------------------------------------------------ GQA

def gqa_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, *, scale: float | None = None,
                  cu_seqlens: np.ndarray | None = None) -> np.ndarray:
    """Causal grouped-query attention in fp64.

    q [B, Hq, T, D], k/v [B, Hkv, T, D] (any float dtype) -> fp64 [B, Hq, T, D].
    Query head h reads KV head h // (Hq // Hkv) (ref: src/decider/native_gqa_kernel.py:39-41);
    key j visible to query i iff j <= i within the same request; this is the
    reference's fp32 MATH-SDPA oracle with enable_gqa=True
    (ref: experiments/native_gqa/bench_native_gqa.py:46-48), in fp64.
    """
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    group = Hq // Hkv
    if scale is None:
        scale = D ** -0.5
    if cu_seqlens is None:
        bounds = [(b, 0, T) for b in range(B)]
    else:
        cu = np.asarray(cu_seqlens, np.int64)
        bounds = [(0, int(cu[i]), int(cu[i + 1])) for i in range(cu.size - 1)]
    out = np.zeros((B, Hq, T, D), np.float64)
    for b, s0, s1 in bounds:
        n = s1 - s0
        if n == 0:
            continue
        mask = np.tril(np.ones((n, n), bool))
        for h in range(Hq):
            kh = h // group
            s = q[b, h, s0:s1] @ k[b, kh, s0:s1].T * scale
            s = np.where(mask, s, -np.inf)
            s = s - s.max(axis=1, keepdims=True)
            p = np.exp(s)
            p /= p.sum(axis=1, keepdims=True)
            out[b, h, s0:s1] = p @ v[b, kh, s0:s1]
    return out


# ---------------------------------------------------------------- readout

def attn_prologue(x_bits: np.ndarray, weight, cos_bits: np.ndarray | None, sin_bits: np.ndarray | None,
                  eps: float = 1e-6, gain_offset: bool = True) -> np.ndarray:
    """Per-head RMSNorm + partial rotary embedding of x [B, T, H, 128] (bf16 bits), bit-exact
    restatement of the GPU kernel (C oracle); weight [128] (uint16 bf16 bits or float32),
    cos / sin [B, T, R] bf16 bits or None.  Returns bf16 bits shaped like x."""
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    B, T, H, D = x.shape
    if D != 128:
        raise ValueError("head_dim must be 128")
    w = np.ascontiguousarray(weight)
    w_dtype = 1 if w.dtype == np.float32 else 0
    if w_dtype == 0:
        w = w.astype(np.uint16)
    rot = 0 if cos_bits is None else cos_bits.shape[-1]
    c = None if cos_bits is None else np.ascontiguousarray(cos_bits, dtype=np.uint16)
    s = None if sin_bits is None else np.ascontiguousarray(sin_bits, dtype=np.uint16)
    out = np.empty_like(x)
    rc = _lib().fd_oracle_attn_prologue(_ptr(x), B * T * H, H, _ptr(w), w_dtype, int(gain_offset), eps,
                                        _ptr(c), _ptr(s), rot, _ptr(out))
    if rc:
        raise ValueError("fd_oracle_attn_prologue rejected its arguments")
    return out


def attn_prologue_f64(x_bits: np.ndarray, weight, cos_bits=None, sin_bits=None, eps: float = 1e-6,
                      gain_offset: bool = True) -> np.ndarray:
    """The same prologue in float64 without intermediate roundings (closed form)."""
    x = bf16_to_f32(x_bits).astype(np.float64)
    w = np.asarray(weight, np.float64) if np.asarray(weight).dtype != np.uint16 else \
        bf16_to_f32(weight).astype(np.float64)
    g = 1.0 + w if gain_offset else w
    y = x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * g
    if cos_bits is not None:
        R = cos_bits.shape[-1]
        c = bf16_to_f32(cos_bits).astype(np.float64)[:, :, None, :]
        s = bf16_to_f32(sin_bits).astype(np.float64)[:, :, None, :]
        yr = y[..., :R]
        rh = np.concatenate([-yr[..., R // 2:], yr[..., :R // 2]], axis=-1)
        y = np.concatenate([yr * c + rh * s, y[..., R:]], axis=-1)
    return y


def slot_readout(hidden_bits: np.ndarray, norm_weight, letters_bits: np.ndarray, rows, positions, nopts=None,
                 eps: float = 1e-6, temperature: float = 1.0, gain_offset: bool = True):
    """Slot-only readout in float64 (ref: src/decider/slot_projection.py:6-21 with the model's final
    Qwen3_5RMSNorm, then src/decider/engine.py:48-56): y = bf16(x / sqrt(mean(x^2) + eps) * (1 + w)) at
    each slot, logits = bf16(y . letters), probs = softmax(logits[:nopts] / temperature).
    hidden [B, T, H] and letters [K, H] bf16 bits; norm_weight float [H].  Returns (logits, probs)."""
    x = bf16_to_f32(hidden_bits[np.asarray(rows), np.asarray(positions)]).astype(np.float64)   # [N, H]
    w = np.asarray(norm_weight, np.float64)
    g = 1.0 + w if gain_offset else w
    y = x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * g
    y = bf16_to_f32(_f64_to_bf16(y)).astype(np.float64)
    lg = y @ bf16_to_f32(letters_bits).astype(np.float64).T
    lg = bf16_to_f32(_f64_to_bf16(lg)).astype(np.float64)
    K = lg.shape[1]
    n = np.full(lg.shape[0], K) if nopts is None else np.asarray(nopts)
    z = np.where(np.arange(K)[None, :] < n[:, None], lg / temperature, -np.inf)
    p = np.exp(z - z.max(axis=1, keepdims=True))
    return lg, p / p.sum(axis=1, keepdims=True)


def gated_rmsnorm(x_bits: np.ndarray, z_bits: np.ndarray, weight, eps: float = 1e-6) -> np.ndarray:
    """transformers' Qwen3_5RMSNormGated on bf16 rows in float64 with its bf16 roundings
    (y = bf16(x / sqrt(mean(x^2) + eps)); y2 = bf16(w * y) for a bf16 weight, w * y for fp32;
    out = y2 * silu(z)); returns the value before its final bf16 rounding."""
    x = bf16_to_f32(x_bits).astype(np.float64)
    z = bf16_to_f32(z_bits).astype(np.float64)
    y = bf16_to_f32(_f64_to_bf16(x / np.sqrt((x * x).mean(-1, keepdims=True) + eps))).astype(np.float64)
    w = np.asarray(weight)
    if w.dtype == np.uint16:
        y2 = bf16_to_f32(_f64_to_bf16(bf16_to_f32(w).astype(np.float64) * y)).astype(np.float64)
    else:
        y2 = w.astype(np.float64) * y
    return y2 * (z / (1.0 + np.exp(-z)))


def silu_mul(gate_up_bits: np.ndarray) -> np.ndarray:
    """The MLP's silu(gate) * up on a combined [..., 2I] bf16 projection: bf16(silu(g)) * u in
    float64 (before the final bf16 rounding)."""
    gu = bf16_to_f32(gate_up_bits).astype(np.float64)
    I = gu.shape[-1] // 2
    g, u = gu[..., :I], gu[..., I:]
    return bf16_to_f32(_f64_to_bf16(g / (1.0 + np.exp(-g)))).astype(np.float64) * u


def gate_transform(a_bits: np.ndarray, b_bits: np.ndarray, a_log, dt_bias) -> tuple[np.ndarray, np.ndarray]:
    """Gated-DeltaNet gate transform in float64 (ref: src/decider/unpack_gate_transform_kernel.py:69-88;
    eager form ref: src/decider/packed_conv.py:49-53): g = -exp(a_log) * softplus(a + dt_bias) with
    softplus(x) = x if x > 20 else log1p(exp(x)), and beta = sigmoid(b) (before its bf16 rounding).
    a, b: bf16 bits [..., H]; a_log, dt_bias: float [H] (bf16 parameters already widened)."""
    # the eager sum a.float() + dt_bias is one fp32 addition; the rest is exact here
    x = (bf16_to_f32(a_bits) + np.asarray(dt_bias, np.float32)).astype(np.float64)
    sp = np.where(x > 20, x, np.log1p(np.exp(np.minimum(x, 20.0))))
    g = -np.exp(np.asarray(a_log, np.float64)) * sp
    beta = 1.0 / (1.0 + np.exp(-bf16_to_f32(b_bits).astype(np.float64)))
    return g, beta


def decide(logits: np.ndarray, nopts) -> tuple[np.ndarray, np.ndarray]:
    """Masked softmax over the first nopts[i] letters of each slot, then argmax.

    Restates ref: src/decider/engine.py:48-56 (gather, mask >= nopts to -inf,
    softmax at temperature 1, ref: src/decider/temperature.py:136-144) and the
    decision ref: src/decider/infer.py:148-151.  logits [N, K] -> (choice [N], probs [N, K]).
    """
    lg = np.asarray(logits, np.float64)
    nopts = np.asarray(nopts)
    mask = np.arange(lg.shape[1])[None, :] >= nopts[:, None]
    lg = np.where(mask, -np.inf, lg)
    lg = lg - lg.max(axis=1, keepdims=True)
    p = np.exp(lg)
    p /= p.sum(axis=1, keepdims=True)
    return p.argmax(axis=1), p
