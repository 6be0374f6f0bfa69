"""CPU oracle for the DiT attention hot path -- TEST INFRASTRUCTURE ONLY.

numpy front end over ``oracle/liboracle.so`` (the C restatement in ``oracle/oracle.c``).
Only ``tests/``, ``__graft_entry__.smoke()`` and the CPU-baseline leg of ``bench.py`` import
this module, and only as the checker.  The product library never routes through it.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int32)
_i8p = ctypes.POINTER(ctypes.c_int8)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_i64 = ctypes.c_int64


class OrcAttn(ctypes.Structure):
    _fields_ = [
        ("B", ctypes.c_int), ("Lq", ctypes.c_int), ("Lk", ctypes.c_int), ("H", ctypes.c_int),
        ("D", ctypes.c_int), ("group", ctypes.c_int),
        ("q", _f32p), ("k", _f32p), ("v", _f32p), ("o", _f32p),
        ("ldq", _i64), ("ldk", _i64), ("ldv", _i64), ("ldo", _i64),
        ("q_off", _i64), ("k_off", _i64), ("v_off", _i64), ("o_off", _i64),
        ("q_bs", _i64), ("k_bs", _i64), ("v_bs", _i64), ("o_bs", _i64),
        ("scale", ctypes.c_float), ("kv_len", _i32p),
    ]


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"oracle not built: {path} (run __graft_entry__.build())")
        L = ctypes.CDLL(path)
        L.orc_randn.argtypes = [ctypes.c_uint64, _i64, _f32p]
        L.orc_mt19937.argtypes = [ctypes.c_uint32, _i64, _u32p]
        L.orc_dit_rope_angles.argtypes = [ctypes.c_int, ctypes.c_int, _f32p]
        L.orc_rope_table.argtypes = [_f32p, _i64, ctypes.c_int, _f32p]
        L.orc_qk_norm_rope.argtypes = [_f32p, _i64, ctypes.c_int, ctypes.c_int, _i64, _f32p, _f32p, _f32p, _i64, ctypes.c_float]
        L.orc_rmsnorm.argtypes = [_f32p, _f32p, _f32p, _i64, ctypes.c_int, ctypes.c_float]
        L.orc_rope.argtypes = [_f32p, _f32p, _i64, ctypes.c_int, ctypes.c_int, _i64, _i64, _i64]
        L.orc_hadamard256.argtypes = [_f32p, _f32p, _i64]
        L.orc_layernorm_mod.argtypes = [_f32p, _f32p, _f32p, _i64, ctypes.c_int, _i64, _i64, ctypes.c_float, ctypes.c_int]
        for name in ("orc_attention_f64", "orc_attention_wgsl", "orc_attention_bf16"):
            getattr(L, name).argtypes = [ctypes.POINTER(OrcAttn)]
        L.orc_bf16_round.argtypes = [ctypes.c_float]
        L.orc_bf16_round.restype = ctypes.c_float
        L.orc_token_quant.argtypes = [_f32p, _i64, ctypes.c_int, _i8p, _f32p]
        L.orc_gemm_i8.argtypes = [_i8p, _i8p, _i64, ctypes.c_int, ctypes.c_int, _i32p]
        L.orc_fp8e4m3.argtypes = [ctypes.c_uint8]
        L.orc_fill_random.argtypes = [ctypes.c_void_p, _i64, ctypes.c_int, ctypes.c_uint64, ctypes.c_float, ctypes.c_float]
        L.orc_channel_norm.argtypes = [_f32p, _f32p, _f32p, _i64, ctypes.c_int, ctypes.c_int]
        L.orc_splitmix64_next.argtypes = [ctypes.c_uint64]
        L.orc_splitmix64_next.restype = ctypes.c_uint64
        L.orc_fp8e4m3.restype = ctypes.c_float
        L.orc_w4_decode.argtypes = [_u8p, _u8p, _f32p, ctypes.c_int, ctypes.c_int, _i8p]
        L.orc_linear_epilogue.argtypes = [_i32p, _i64, ctypes.c_int, _f32p, _f32p, _f32p, ctypes.c_int, ctypes.c_int, _f32p, _i64, _f32p, _i64,
                                          _f32p]
        L.orc_gelu.argtypes = [ctypes.c_float]
        L.orc_gelu.restype = ctypes.c_float
        L.orc_silu.argtypes = [ctypes.c_float]
        L.orc_silu.restype = ctypes.c_float
        _LIB = L
    return _LIB


def _p(a, t):
    return a.ctypes.data_as(t) if a is not None else None


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ------------------------------------------------------------------ RNG

def randn(seed: int, n: int) -> np.ndarray:
    """torch.manual_seed(seed); torch.randn(n) (app/rng.js:55-66)."""
    out = np.empty(n, np.float32)
    lib().orc_randn(seed, n, _p(out, _f32p))
    return out


def mt19937(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.uint32)
    lib().orc_mt19937(seed, n, _p(out, _u32p))
    return out


# ------------------------------------------------------------------ RoPE

def dit_rope_angles(Hp: int, Wp: int) -> np.ndarray:
    out = np.empty((Hp * Wp, 64), np.float32)
    lib().orc_dit_rope_angles(Hp, Wp, _p(out, _f32p))
    return out


def rope_table(angles: np.ndarray) -> np.ndarray:
    """cos block then sin block, flat [2*L*half]; sin_off = L*half (common.js:3-12)."""
    a = _c(angles, np.float32)
    L, half = a.shape
    out = np.empty(2 * L * half, np.float32)
    lib().orc_rope_table(_p(a, _f32p), L, half, _p(out, _f32p))
    return out


def dit_rope_table(Hp: int, Wp: int) -> np.ndarray:
    return rope_table(dit_rope_angles(Hp, Wp))


# ------------------------------------------------------------------ row ops

def qk_norm_rope(qkv, L, H, D, ld, qn, kn, cs, sin_off, eps=1e-6):
    x = np.array(qkv, dtype=np.float32, copy=True, order="C")
    qn, kn, cs = _c(qn, np.float32), _c(kn, np.float32), _c(cs, np.float32)
    lib().orc_qk_norm_rope(_p(x, _f32p), L, H, D, ld, _p(qn, _f32p), _p(kn, _f32p), _p(cs, _f32p), sin_off, eps)
    return x


def rmsnorm(x, w, cols, eps=1e-6):
    x = _c(x, np.float32)
    w = _c(w, np.float32)
    y = np.empty_like(x)
    lib().orc_rmsnorm(_p(x, _f32p), _p(w, _f32p), _p(y, _f32p), x.size // cols, cols, eps)
    return y


def rope(x, cs, L, H, D, sin_off, row_stride=None, col_off=0):
    y = np.array(x, dtype=np.float32, copy=True, order="C")
    cs = _c(cs, np.float32)
    lib().orc_rope(_p(y, _f32p), _p(cs, _f32p), L, H, D, sin_off, row_stride or H * D, col_off)
    return y


def hadamard256(x):
    x = _c(x, np.float32)
    y = np.empty_like(x)
    lib().orc_hadamard256(_p(x, _f32p), _p(y, _f32p), x.size)
    return y


def layernorm_mod(x, mod, shift_off, scale_off, cols, rotate=False, eps=1e-6):
    x = _c(x, np.float32)
    mod = _c(mod, np.float32)
    y = np.empty_like(x)
    lib().orc_layernorm_mod(_p(x, _f32p), _p(mod, _f32p), _p(y, _f32p), x.size // cols, cols, shift_off, scale_off, eps, int(rotate))
    return y


# ------------------------------------------------------------------ attention

def attention(kind, q, k, v, *, B, Lq, Lk, H, D, ldq, ldk, ldv, q_off=0, k_off=0, v_off=0,
              q_bs=None, k_bs=None, v_bs=None, group=1, scale=None, kv_len=None):
    """kind: 'f64' | 'wgsl' | 'bf16'.  Returns O [B, Lq, H*D] fp32."""
    q, k, v = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32)
    o = np.zeros((B, Lq, H * D), np.float32)
    kl = _c(kv_len, np.int32) if kv_len is not None else None
    a = OrcAttn(B=B, Lq=Lq, Lk=Lk, H=H, D=D, group=group,
                q=_p(q, _f32p), k=_p(k, _f32p), v=_p(v, _f32p), o=_p(o, _f32p),
                ldq=ldq, ldk=ldk, ldv=ldv, ldo=H * D, q_off=q_off, k_off=k_off, v_off=v_off, o_off=0,
                q_bs=q_bs if q_bs is not None else Lq * ldq,
                k_bs=k_bs if k_bs is not None else Lk * ldk,
                v_bs=v_bs if v_bs is not None else Lk * ldv,
                o_bs=Lq * H * D,
                scale=np.float32(scale if scale is not None else 1.0 / np.sqrt(D)),
                kv_len=_p(kl, _i32p))
    getattr(lib(), "orc_attention_" + kind)(ctypes.byref(a))
    return o


def bf16_round(x):
    x = _c(x, np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    nan = np.isnan(x)
    out = r.view(np.float32).copy()
    out[nan] = np.nan
    return out


# ------------------------------------------------------------------ quantized linears

def token_quant(x):
    x = _c(x, np.float32)
    M, K = x.shape
    q = np.empty((M, K), np.int8)
    s = np.empty(M, np.float32)
    lib().orc_token_quant(_p(x, _f32p), M, K, _p(q, _i8p), _p(s, _f32p))
    return q, s


def gemm_i8(qx, qw):
    qx, qw = _c(qx, np.int8), _c(qw, np.int8)
    M, K = qx.shape
    N = qw.shape[0]
    acc = np.empty((M, N), np.int32)
    lib().orc_gemm_i8(_p(qx, _i8p), _p(qw, _i8p), M, N, K, _p(acc, _i32p))
    return acc


def fp8e4m3(b: int) -> float:
    return lib().orc_fp8e4m3(b)


def w4_decode(codes, srel, codebook, N, K):
    codes, srel = _c(codes, np.uint8), _c(srel, np.uint8)
    cb = _c(codebook, np.float32)
    out = np.empty((N, K), np.int8)
    lib().orc_w4_decode(_p(codes, _u8p), _p(srel, _u8p), _p(cb, _f32p), N, K, _p(out, _i8p))
    return out


def linear_epilogue(acc, sx, sw, *, bias=None, act=0, epi=0, gate=None, g_off=0, c=None, add=None):
    """add: optional [M, N] term after the bias (the LoRA delta, gemm.js:189)."""
    acc = _c(acc, np.int32)
    M, N = acc.shape
    sx = _c(sx, np.float32) if sx is not None else None
    sw = _c(sw, np.float32)
    bias = _c(bias, np.float32) if bias is not None else None
    gate = _c(gate, np.float32) if gate is not None else None
    add = _c(add, np.float32) if add is not None else None
    out = np.zeros((M, N), np.float32) if c is None else np.array(c, dtype=np.float32, copy=True, order="C")
    lib().orc_linear_epilogue(_p(acc, _i32p), M, N, _p(sx, _f32p), _p(sw, _f32p), _p(bias, _f32p), act, epi,
                              _p(gate, _f32p), g_off, _p(out, _f32p), N, _p(add, _f32p))
    return out


def gelu(x: float) -> float:
    return lib().orc_gelu(x)


def silu(x: float) -> float:
    return lib().orc_silu(x)


FILL_KINDS = {"u8": (0, np.uint8), "i8n": (1, np.int8), "f32": (2, np.float32), "bf16": (3, np.uint16),
              "f32n": (4, np.float32)}


def fill_random(n, kind, seed, lo, hi):
    """The seeded synthetic fill of anima_fill_random (bf16 as its uint16 bit patterns)."""
    k, dt = FILL_KINDS[kind]
    out = np.empty(n, dt)
    lib().orc_fill_random(out.ctypes.data_as(ctypes.c_void_p), n, k, seed, lo, hi)
    return out


def splitmix64_next(state):
    return int(lib().orc_splitmix64_next(state))


def channel_norm(x, gamma, cols, silu=False):
    """Wan VAE channel norm (app/gpu/kernels.js:62-89 mode 1) over rows of `cols`."""
    x = _c(x, np.float32)
    g = _c(gamma, np.float32)
    y = np.empty_like(x)
    lib().orc_channel_norm(_p(x, _f32p), _p(g, _f32p), _p(y, _f32p), x.size // cols, cols, int(silu))
    return y
