"""Python binding of libanima.so (the C ABI in include/anima.h), used by the tests and bench.

The product's host side is the Node N-API addon under js/; this module is a second thin host
over the same C ABI.  It never computes anything itself: if libanima.so is missing or cannot
be loaded, every entry point raises.
"""

from __future__ import annotations

import ctypes
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libanima.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "anima.h")

ANIMA_OK = 0
PREC_BF16 = 0
PREC_FP32 = 1
W_BF16, W_I8, W_W4, W_F32, W_F32S3 = 0, 1, 2, 3, 4
W4_GRID_SCRATCH, W4_IN_GEMM = 0, 1
ACT = {"none": 0, "gelu": 1, "silu": 2}
EPI_STORE, EPI_RESID, EPI_GATED = 0, 1, 2
EW = {"silu_mul": 0, "add": 1, "silu": 2, "copy": 3}

_i64 = ctypes.c_int64
_vp = ctypes.c_void_p
_LIB = None


class AnimaError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"anima error {code}: {msg}")
        self.code = code


class AttnDesc(ctypes.Structure):
    _fields_ = [
        ("B", ctypes.c_int), ("Lq", ctypes.c_int), ("Lk", ctypes.c_int), ("H", ctypes.c_int), ("D", ctypes.c_int),
        ("group", ctypes.c_int),
        ("q", _vp), ("ldq", _i64), ("q_off", _i64), ("q_bstride", _i64),
        ("k", _vp), ("ldk", _i64), ("k_off", _i64), ("k_bstride", _i64),
        ("v", _vp), ("ldv", _i64), ("v_off", _i64), ("v_bstride", _i64),
        ("o", _vp), ("ldo", _i64), ("o_off", _i64), ("o_bstride", _i64),
        ("scale", ctypes.c_float),
        ("kv_len", ctypes.POINTER(ctypes.c_int)),
        ("precision", ctypes.c_int),
        ("q_norm", _vp), ("k_norm", _vp), ("rope_cs", _vp), ("rope_sin_off", _i64),
        ("eps", ctypes.c_float),
        ("causal", ctypes.c_int),
        ("kv_prep", _vp),
        ("kv_prep_bytes", _i64),
        ("q_prep", _vp),
        ("o_bf16", ctypes.c_int),
    ]


class ConvDesc(ctypes.Structure):
    _fields_ = [("B", ctypes.c_int), ("H", ctypes.c_int), ("W", ctypes.c_int), ("cin", ctypes.c_int),
                ("cout", ctypes.c_int), ("up", ctypes.c_int), ("x", _vp), ("w", _vp), ("bias", _vp), ("out", _vp),
                ("resid", ctypes.c_int), ("precision", ctypes.c_int)]


class Weight(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int), ("N", ctypes.c_int), ("K", ctypes.c_int), ("w", _vp), ("scale", _vp),
                ("srel", _vp), ("codebook", _vp), ("bias", _vp)]


class LinearDesc(ctypes.Structure):
    _fields_ = [("M", _i64), ("W", ctypes.POINTER(Weight)), ("x", _vp), ("ldx", _i64), ("x_rotated", ctypes.c_int),
                ("xq", _vp), ("xs", _vp), ("out", _vp), ("ldc", _i64), ("alpha", ctypes.c_float),
                ("act", ctypes.c_int), ("epilogue", ctypes.c_int), ("gate", _vp), ("gate_off", _i64),
                ("acc_out", _vp), ("add", _vp), ("ld_add", _i64), ("lora_xa", _vp), ("ld_lora_xa", _i64),
                ("lora_b", _vp), ("lora_r", ctypes.c_int), ("lora_cols", ctypes.c_int)]


SAMPLER = {"euler": 0, "euler_a": 1, "dpmpp_2m": 2, "er_sde": 3}


class SamplerDesc(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int), ("n", _i64), ("x", _vp), ("v", _vp), ("v_uncond", _vp),
                ("cfg", ctypes.c_double), ("sigma", ctypes.c_double), ("final_step", ctypes.c_int),
                ("stage", ctypes.c_int), ("den_out", _vp), ("old", _vp), ("old_d", _vp), ("eps", _vp),
                ("c", ctypes.c_double * 10)]


class Limits(ctypes.Structure):
    _fields_ = [("max_buffer_size", _i64), ("max_binding_size", _i64), ("total_memory", _i64),
                ("free_memory", _i64), ("workgroup_storage_size", ctypes.c_int32),
                ("max_workgroup_size", ctypes.c_int32), ("max_workgroups_per_dimension", ctypes.c_int32),
                ("compute_units", ctypes.c_int32), ("wavefront_size", ctypes.c_int32), ("clock_khz", ctypes.c_int32),
                ("arch", ctypes.c_char * 64)]


class QkvDesc(ctypes.Structure):
    _fields_ = [("B", ctypes.c_int), ("L", ctypes.c_int), ("H", ctypes.c_int), ("k_norm", _vp), ("rope_cs", _vp),
                ("rope_sin_off", _i64), ("eps", ctypes.c_float), ("kv_prep", _vp), ("kv_prep_bytes", _i64),
                ("q_norm", _vp), ("q_prep", _vp), ("q_scale", ctypes.c_float)]


ABI_STRUCTS = {"anima_attn_desc": AttnDesc, "anima_linear_desc": LinearDesc, "anima_weight": Weight,
               "anima_sampler_desc": SamplerDesc, "anima_conv_desc": ConvDesc, "anima_limits": Limits,
               "anima_qkv_desc": QkvDesc}


def abi_mismatches(L):
    """Differences between the ctypes restatement of the descriptor structs above and the
    library's own layout (anima_abi_offset): sizes and the offset of every field."""
    bad = []
    for cname, S in ABI_STRUCTS.items():
        size = L.anima_abi_offset(cname.encode(), None)
        if size != ctypes.sizeof(S):
            bad.append(f"sizeof({cname}) = {size}, binding {ctypes.sizeof(S)}")
        for fname, _ in S._fields_:
            off = L.anima_abi_offset(cname.encode(), fname.encode())
            if off != getattr(S, fname).offset:
                bad.append(f"{cname}.{fname} at {off}, binding {getattr(S, fname).offset}")
    return bad


def check_abi(L):
    bad = abi_mismatches(L)
    if bad:
        raise RuntimeError("the ctypes binding does not match libanima.so's structs: " + "; ".join(bad))


def lib():
    """Loads libanima.so (raises if it is not built, or if its descriptor layouts differ from the
    structs restated here)."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run __graft_entry__.build()")
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.POINTER
        L.anima_abi_offset.argtypes = [ctypes.c_char_p, ctypes.c_char_p]
        L.anima_abi_offset.restype = _i64
        check_abi(L)
        L.anima_init.argtypes = [ctypes.c_int, P(_vp)]
        L.anima_destroy.argtypes = [_vp]
        L.anima_last_error.argtypes = [_vp]
        L.anima_last_error.restype = ctypes.c_char_p
        for n in ("anima_sync", "anima_flush", "anima_pool_trim", "anima_profile_reset", "anima_timer_start"):
            getattr(L, n).argtypes = [_vp]
        L.anima_mem_stats.argtypes = [_vp, P(ctypes.c_uint64), P(ctypes.c_uint64), P(ctypes.c_uint64)]
        L.anima_device_limits.argtypes = [_vp, P(Limits)]
        L.anima_set_w4_path.argtypes = [_vp, ctypes.c_int]
        L.anima_alloc.argtypes = [_vp, ctypes.c_size_t, P(_vp)]
        L.anima_free.argtypes = [_vp, _vp]
        for n in ("anima_h2d", "anima_d2h", "anima_d2d"):
            getattr(L, n).argtypes = [_vp, _vp, _vp, ctypes.c_size_t]
        L.anima_mark.argtypes = [_vp, P(ctypes.c_uint64)]
        L.anima_wait_mark.argtypes = [_vp, ctypes.c_uint64]
        L.anima_profile_enable.argtypes = [_vp, ctypes.c_int]
        L.anima_profile_report.argtypes = [_vp, ctypes.c_char_p, ctypes.c_size_t]
        L.anima_timer_stop.argtypes = [_vp, P(ctypes.c_float)]
        L.anima_attention.argtypes = [_vp, P(AttnDesc)]
        L.anima_linear_qkv.argtypes = [_vp, P(LinearDesc), P(QkvDesc)]
        L.anima_attention_prepare_kv.argtypes = [_vp, P(AttnDesc), _vp]
        L.anima_attention_kv_bytes.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.anima_attention_kv_bytes.restype = _i64
        L.anima_qk_norm_rope.argtypes = [_vp, _vp, _i64, ctypes.c_int, ctypes.c_int, _i64, _vp, _vp, _vp, _i64, ctypes.c_float]
        L.anima_rmsnorm.argtypes = [_vp, _vp, _vp, _vp, _i64, ctypes.c_int, ctypes.c_float]
        L.anima_rope.argtypes = [_vp, _vp, _vp, _i64, ctypes.c_int, ctypes.c_int, _i64, _i64, _i64]
        L.anima_hadamard.argtypes = [_vp, _vp, _vp, _i64]
        L.anima_quant_rows.argtypes = [_vp, _vp, _i64, ctypes.c_int, ctypes.c_int, _vp, _vp]
        L.anima_quant_rows_act.argtypes = [_vp, _vp, _i64, ctypes.c_int, ctypes.c_int, ctypes.c_int, _vp, _vp]
        L.anima_quant_rows_bf16.argtypes = [_vp, _vp, _i64, ctypes.c_int, ctypes.c_int, _vp, _vp]
        L.anima_layernorm_mod.argtypes = [_vp, _vp, _vp, _i64, _i64, _i64, ctypes.c_int, ctypes.c_float, ctypes.c_int,
                                          _vp, _vp, _vp]
        L.anima_elementwise.argtypes = [_vp, ctypes.c_int, _vp, _vp, _vp, _i64]
        L.anima_zero.argtypes = [_vp, _vp, _i64]
        L.anima_linear_grouped_bf16.argtypes = [_vp, ctypes.c_int, _i64, ctypes.c_int, ctypes.c_int, _vp, _i64, _i64, _vp,
                                                 _i64, _vp, _i64, _vp, _i64, _i64]
        L.anima_gemv_grouped_f32.argtypes = [_vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, _vp, _i64, _vp, _i64, _vp,
                                             _i64, ctypes.c_float, ctypes.c_int]
        L.anima_patchify.argtypes = [_vp, _vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, _vp]
        L.anima_unpatchify.argtypes = [_vp, _vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, _vp]
        L.anima_linear.argtypes = [_vp, ctypes.POINTER(LinearDesc)]
        L.anima_weight_unpack_w4.argtypes = [_vp, ctypes.POINTER(Weight), _vp]
        L.anima_sampler_step.argtypes = [_vp, ctypes.POINTER(SamplerDesc)]
        L.anima_split3_bf16.argtypes = [_vp, _vp, _vp, _i64]
        L.anima_attention_noalloc.argtypes = [_vp, ctypes.POINTER(AttnDesc)]
        L.anima_attention_noalloc_scratch_bytes.argtypes = []
        L.anima_attention_noalloc_scratch_bytes.restype = _i64
        L.anima_conv3x3.argtypes = [_vp, ctypes.POINTER(ConvDesc)]
        L.anima_channel_norm.argtypes = [_vp, _vp, _vp, _vp, _i64, ctypes.c_int, ctypes.c_int]
        L.anima_fill_random.argtypes = [_vp, _vp, _i64, ctypes.c_int, ctypes.c_uint64, ctypes.c_float, ctypes.c_float]
        L.anima_graph_begin.argtypes = [_vp]
        L.anima_graph_end.argtypes = [_vp, P(_vp)]
        L.anima_graph_launch.argtypes = [_vp, _vp]
        L.anima_graph_destroy.argtypes = [_vp, _vp]
        _LIB = L
    return _LIB


def declared_symbols():
    """Entry points declared in include/anima.h."""
    import re

    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w[\w\s\*]*?\b(anima_\w+)\s*\(", text, re.M)))


class DeviceBuffer:
    """A pooled device allocation (Tensor of app/gpu/device.js:10-24, untyped)."""

    def __init__(self, ctx, nbytes, shape=None, dtype=None):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        self.shape = shape
        self.dtype = np.dtype(dtype) if dtype is not None else None
        p = _vp()
        ctx._check(lib().anima_alloc(ctx.h, max(1, self.nbytes), ctypes.byref(p)))
        self.ptr = p.value

    def release(self):
        if self.ptr is not None:
            self.ctx._check(lib().anima_free(self.ctx.h, self.ptr))
            self.ptr = None

    def numpy(self):
        out = np.empty(self.shape, self.dtype)
        self.ctx._check(lib().anima_d2h(self.ctx.h, out.ctypes.data, self.ptr, out.nbytes))
        return out

    def write(self, arr):
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes
        self.ctx._check(lib().anima_h2d(self.ctx.h, self.ptr, arr.ctypes.data, arr.nbytes))


class Context:
    """One HIP device + stream (GPU of app/gpu/device.js:59-232)."""

    def __init__(self, device=0):
        h = _vp()
        rc = lib().anima_init(device, ctypes.byref(h))
        if rc != ANIMA_OK:
            raise AnimaError(rc, lib().anima_last_error(None).decode())
        self.h = h.value

    def close(self):
        if self.h:
            lib().anima_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def _check(self, rc):
        if rc != ANIMA_OK:
            raise AnimaError(rc, lib().anima_last_error(self.h).decode())
        return rc

    def last_error(self):
        return lib().anima_last_error(self.h).decode()

    # ---- memory
    def empty(self, shape, dtype=np.float32):
        shape = tuple(int(s) for s in np.atleast_1d(shape))
        return DeviceBuffer(self, int(np.prod(shape)) * np.dtype(dtype).itemsize, shape, dtype)

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        b = DeviceBuffer(self, arr.nbytes, arr.shape, arr.dtype)
        b.write(arr)
        return b

    def sync(self):
        self._check(lib().anima_sync(self.h))

    def mark(self):
        """A point in the stream; wait_mark(t) returns once the work enqueued before it is done."""
        t = ctypes.c_uint64()
        self._check(lib().anima_mark(self.h, ctypes.byref(t)))
        return t.value

    def wait_mark(self, ticket):
        self._check(lib().anima_wait_mark(self.h, ticket))

    def mem_stats(self):
        a, p, q = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
        self._check(lib().anima_mem_stats(self.h, ctypes.byref(a), ctypes.byref(p), ctypes.byref(q)))
        return {"allocated": a.value, "peak": p.value, "pooled": q.value}

    def set_w4_path(self, path):
        """W4_GRID_SCRATCH (default) or W4_IN_GEMM for the large W4 products (anima_set_w4_path)."""
        self._check(lib().anima_set_w4_path(self.h, path))

    def limits(self):
        """The device limits (anima_device_limits), as a dict."""
        d = Limits()
        self._check(lib().anima_device_limits(self.h, ctypes.byref(d)))
        out = {f: getattr(d, f) for f, _ in Limits._fields_}
        out["arch"] = d.arch.decode()
        return out

    def trim(self):
        self._check(lib().anima_pool_trim(self.h))

    # ---- profiling / timing
    def profile(self, on=True):
        self._check(lib().anima_profile_enable(self.h, int(on)))

    def profile_reset(self):
        self._check(lib().anima_profile_reset(self.h))

    def profile_report(self):
        buf = ctypes.create_string_buffer(1 << 16)
        self._check(lib().anima_profile_report(self.h, buf, len(buf)))
        return json.loads(buf.value.decode())

    def timer_start(self):
        self._check(lib().anima_timer_start(self.h))

    def timer_stop(self):
        ms = ctypes.c_float()
        self._check(lib().anima_timer_stop(self.h, ctypes.byref(ms)))
        return ms.value

    # ---- recorded submission (HIP graphs)
    def graph_begin(self):
        """Starts capturing this context's work (anima_graph_begin)."""
        self._check(lib().anima_graph_begin(self.h))

    def graph_end(self):
        """Ends the capture and returns a replayable graph handle."""
        g = _vp()
        self._check(lib().anima_graph_end(self.h, ctypes.byref(g)))
        return g.value

    def graph_launch(self, g):
        self._check(lib().anima_graph_launch(self.h, g))

    def graph_destroy(self, g):
        self._check(lib().anima_graph_destroy(self.h, g))

    # ---- ops
    def attention(self, *, q, k, v, o, B, Lq, Lk, H, D, ldq, ldk, ldv, ldo=None, q_off=0, k_off=0, v_off=0,
                  o_off=0, q_bstride=None, k_bstride=None, v_bstride=None, o_bstride=None, group=1, scale=0.0,
                  kv_len=None, precision=PREC_BF16, q_norm=None, k_norm=None, rope_cs=None, rope_sin_off=0,
                  eps=1e-6, causal=0, kv_prep=None, prepare_into=None, kv_prep_bytes=None, noalloc=False,
                  q_prep=None, o_bf16=False):
        """anima_attention; kv_prep: K/V converted by a call with prepare_into (which runs
        anima_attention_prepare_kv into that buffer instead of the attention).  kv_prep_bytes
        defaults to the size the call's shape and precision take.  noalloc: anima_attention_noalloc
        (the K/V conversion in the library's static scratch, no allocation).  q_prep: Q as
        linear_qkv(q_prep=...) prepared it (then q may be None).  o_bf16: O written as bf16 (o and its
        strides in uint16 elements)."""
        ldo = ldo if ldo is not None else H * D
        kl = (ctypes.c_int * B)(*[int(x) for x in kv_len]) if kv_len is not None else None
        d = AttnDesc(B=B, Lq=Lq, Lk=Lk, H=H, D=D, group=group,
                     q=_ptr(q), ldq=ldq, q_off=q_off, q_bstride=q_bstride if q_bstride is not None else Lq * ldq,
                     k=_ptr(k), ldk=ldk, k_off=k_off, k_bstride=k_bstride if k_bstride is not None else Lk * ldk,
                     v=_ptr(v), ldv=ldv, v_off=v_off, v_bstride=v_bstride if v_bstride is not None else Lk * ldv,
                     o=_ptr(o), ldo=ldo, o_off=o_off, o_bstride=o_bstride if o_bstride is not None else Lq * ldo,
                     scale=scale, kv_len=ctypes.cast(kl, ctypes.POINTER(ctypes.c_int)) if kl is not None else None,
                     precision=precision, q_norm=_ptr(q_norm), k_norm=_ptr(k_norm), rope_cs=_ptr(rope_cs),
                     rope_sin_off=rope_sin_off, eps=eps, causal=causal, kv_prep=_ptr(kv_prep), q_prep=_ptr(q_prep),
                     o_bf16=int(o_bf16),
                     kv_prep_bytes=kv_prep_bytes if kv_prep_bytes is not None else
                     (self.attention_kv_bytes(B, H // max(group, 1), Lk, precision)
                      if (kv_prep is not None or prepare_into is not None) else 0))
        if prepare_into is not None:
            return self._check(lib().anima_attention_prepare_kv(self.h, ctypes.byref(d), _ptr(prepare_into)))
        if noalloc:
            return self._check(lib().anima_attention_noalloc(self.h, ctypes.byref(d)))
        return self._check(lib().anima_attention(self.h, ctypes.byref(d)))

    @staticmethod
    def attention_noalloc_scratch_bytes():
        return lib().anima_attention_noalloc_scratch_bytes()

    @staticmethod
    def attention_kv_bytes(B, Hkv, Lk, precision=PREC_BF16):
        return lib().anima_attention_kv_bytes(B, Hkv, Lk, precision)

    FILL = {"u8": 0, "i8n": 1, "f32": 2, "bf16": 3, "f32n": 4}

    def fill_random(self, dst, n, kind, seed, lo, hi):
        """anima_fill_random: the seeded synthetic fill (kind "u8" / "i8n" / "f32" / "bf16" / "f32n")."""
        return self._check(lib().anima_fill_random(self.h, _ptr(dst), n, self.FILL[kind], seed, lo, hi))

    def conv3x3(self, x, w, out, *, B, H, W, cin, cout, up=False, bias=None, resid=False, precision=PREC_FP32):
        """anima_conv3x3 (output H x W per image; the input is half that with up)."""
        d = ConvDesc(B=B, H=H, W=W, cin=cin, cout=cout, up=int(up), x=_ptr(x), w=_ptr(w), bias=_ptr(bias),
                     out=_ptr(out), resid=int(resid), precision=precision)
        return self._check(lib().anima_conv3x3(self.h, ctypes.byref(d)))

    def channel_norm(self, x, gamma, y, rows, cols, silu=False):
        return self._check(lib().anima_channel_norm(self.h, _ptr(x), _ptr(gamma), _ptr(y), rows, cols, int(silu)))

    def hadamard(self, x, y, n):
        return self._check(lib().anima_hadamard(self.h, _ptr(x), _ptr(y), n))

    def quant_rows(self, x, M, K, rotate, q, s, act="none"):
        if act != "none":
            return self._check(lib().anima_quant_rows_act(self.h, _ptr(x), M, K, ACT[act], int(rotate), _ptr(q),
                                                          _ptr(s)))
        return self._check(lib().anima_quant_rows(self.h, _ptr(x), M, K, int(rotate), _ptr(q), _ptr(s)))

    def quant_rows_bf16(self, x, M, K, rotate, q, s):
        """anima_quant_rows_bf16: quant_rows of bf16 rows (uint16 x)."""
        return self._check(lib().anima_quant_rows_bf16(self.h, _ptr(x), M, K, int(rotate), _ptr(q), _ptr(s)))

    def layernorm_mod(self, x, mod, shift_off, scale_off, rows, cols, rotate=False, y=None, q=None, s=None, eps=1e-6):
        return self._check(lib().anima_layernorm_mod(self.h, _ptr(x), _ptr(mod), shift_off, scale_off, rows, cols, eps,
                                                     int(rotate), _ptr(y), _ptr(q), _ptr(s)))

    def elementwise(self, op, a, b, y, n):
        return self._check(lib().anima_elementwise(self.h, EW[op] if isinstance(op, str) else op, _ptr(a), _ptr(b),
                                                   _ptr(y), n))

    def zero(self, y, n):
        return self._check(lib().anima_zero(self.h, _ptr(y), n))

    def linear_grouped_bf16(self, G, M, N, K, x, ldx, x_gstride, w, w_gstride, bias, bias_gstride, out, ldc,
                            out_gstride):
        return self._check(lib().anima_linear_grouped_bf16(self.h, G, M, N, K, _ptr(x), ldx, x_gstride, _ptr(w),
                                                           w_gstride, _ptr(bias), bias_gstride, _ptr(out), ldc,
                                                           out_gstride))

    def gemv_grouped_f32(self, G, N, K, x, x_gstride, w, w_gstride, y, y_gstride, alpha=0.0, accumulate=False):
        """anima_gemv_grouped_f32: y_g = alpha * W_g x_g (+ y_g) for G groups in one launch."""
        return self._check(lib().anima_gemv_grouped_f32(self.h, G, N, K, _ptr(x), x_gstride, _ptr(w), w_gstride,
                                                        _ptr(y), y_gstride, alpha, int(accumulate)))

    def patchify(self, latents, B, h, w, patches):
        return self._check(lib().anima_patchify(self.h, _ptr(latents), B, h, w, _ptr(patches)))

    def unpatchify(self, o, B, h, w, latents):
        return self._check(lib().anima_unpatchify(self.h, _ptr(o), B, h, w, _ptr(latents)))

    def linear(self, W, M, out, *, x=None, ldx=0, x_rotated=True, xq=None, xs=None, ldc=0, alpha=0.0, act="none",
               epilogue=EPI_STORE, gate=None, gate_off=0, acc_out=None, add=None, ld_add=0, lora_xa=None,
               ld_lora_xa=0, lora_b=None, lora_r=0, lora_cols=0):
        """anima_linear; lora_xa / lora_b / lora_r: the LoRA delta's factors for the quantized
        GEMM's epilogue (A products [M][ld_lora_xa] fp32, B as three bf16 planes [3][N][lora_r]);
        lora_cols > 0: block-diagonal ranks, column n reading xa columns (n // lora_cols) * lora_r
        + k."""
        d = LinearDesc(M=M, W=ctypes.pointer(W), x=_ptr(x), ldx=ldx, x_rotated=int(x_rotated), xq=_ptr(xq),
                       xs=_ptr(xs), out=_ptr(out), ldc=ldc, alpha=alpha, act=ACT[act] if isinstance(act, str) else act,
                       epilogue=epilogue, gate=_ptr(gate), gate_off=gate_off, acc_out=_ptr(acc_out), add=_ptr(add),
                       ld_add=ld_add, lora_xa=_ptr(lora_xa), ld_lora_xa=ld_lora_xa, lora_b=_ptr(lora_b),
                       lora_r=lora_r, lora_cols=lora_cols)
        return self._check(lib().anima_linear(self.h, ctypes.byref(d)))

    def linear_qkv(self, W, M, out, *, B, L, H, k_norm=None, rope_cs=None, rope_sin_off=0, kv_prep=None, eps=1e-6,
                   x=None, ldx=0, x_rotated=True, xq=None, xs=None, ldc=0, alpha=0.0, lora_xa=None, ld_lora_xa=0,
                   lora_b=None, lora_r=0, lora_cols=0, q_norm=None, q_prep=None, q_scale=0.0):
        """anima_linear_qkv: the stacked QKV projection writing Q (fp32) to out and K / V in the
        attention's bf16 operand layout to kv_prep (sized by attention_kv_bytes(B, H, L, bf16));
        lora_*: the LoRA factors as for linear(), added before the K / V conversion; q_prep: Q in the
        attention's prepared bf16 form (q_norm, RoPE, q_scale) instead of fp32 into out (out may then
        be None; with W of H * 128 columns, a Q-only projection)."""
        d = LinearDesc(M=M, W=ctypes.pointer(W), x=_ptr(x), ldx=ldx, x_rotated=int(x_rotated), xq=_ptr(xq),
                       xs=_ptr(xs), out=_ptr(out), ldc=ldc, alpha=alpha, act=0, epilogue=EPI_STORE,
                       lora_xa=_ptr(lora_xa), ld_lora_xa=ld_lora_xa, lora_b=_ptr(lora_b), lora_r=lora_r,
                       lora_cols=lora_cols)
        p = QkvDesc(B=B, L=L, H=H, k_norm=_ptr(k_norm), rope_cs=_ptr(rope_cs), rope_sin_off=rope_sin_off, eps=eps,
                    kv_prep=_ptr(kv_prep), kv_prep_bytes=self.attention_kv_bytes(B, H, L, PREC_BF16) if kv_prep else 0,
                    q_norm=_ptr(q_norm), q_prep=_ptr(q_prep), q_scale=q_scale)
        return self._check(lib().anima_linear_qkv(self.h, ctypes.byref(d), ctypes.byref(p)))

    def weight_unpack_w4(self, W, grid):
        """The int8 grid [N][K] of a W4 weight (anima_weight_unpack_w4)."""
        return self._check(lib().anima_weight_unpack_w4(self.h, ctypes.byref(W), _ptr(grid)))

    def split3_bf16(self, src, dst, n):
        return self._check(lib().anima_split3_bf16(self.h, _ptr(src), _ptr(dst), n))

    def sampler_step(self, kind, n, x, v, *, v_uncond=None, cfg=1.0, sigma, final_step=False, stage=0, den_out=None,
                     old=None, old_d=None, eps=None, c=()):
        cc = (ctypes.c_double * 10)(*[float(t) for t in c])
        d = SamplerDesc(kind=SAMPLER[kind] if isinstance(kind, str) else kind, n=n, x=_ptr(x), v=_ptr(v),
                        v_uncond=_ptr(v_uncond), cfg=cfg, sigma=sigma, final_step=int(final_step), stage=stage,
                        den_out=_ptr(den_out), old=_ptr(old), old_d=_ptr(old_d), eps=_ptr(eps), c=cc)
        return self._check(lib().anima_sampler_step(self.h, ctypes.byref(d)))

    def qk_norm_rope(self, qkv, L, H, D, ld, qn, kn, cs, sin_off, eps=1e-6):
        return self._check(lib().anima_qk_norm_rope(self.h, _ptr(qkv), L, H, D, ld, _ptr(qn), _ptr(kn), _ptr(cs), sin_off, eps))

    def rmsnorm(self, x, w, y, rows, cols, eps=1e-6):
        return self._check(lib().anima_rmsnorm(self.h, _ptr(x), _ptr(w), _ptr(y), rows, cols, eps))

    def rope(self, x, cs, L, H, D, sin_off, row_stride=None, col_off=0):
        return self._check(lib().anima_rope(self.h, _ptr(x), _ptr(cs), L, H, D, sin_off,
                                            row_stride if row_stride is not None else H * D, col_off))


def weight(kind, N, K, w, scale=None, srel=None, codebook=None, bias=None):
    """Linear weight object of app/weights.js:1-4 (device buffers)."""
    return Weight(kind=kind, N=N, K=K, w=_ptr(w), scale=_ptr(scale), srel=_ptr(srel), codebook=_ptr(codebook),
                  bias=_ptr(bias))


def dit_rope_angles(Hp: int, Wp: int) -> np.ndarray:
    """Angles [Hp*Wp][64] of the 3D Cosmos RoPE for one frame (app/models/common.js:31-52):
    slots 0..21 temporal at t=0 (angle 0), 22..42 row * hf[j], 43..63 column * hf[j],
    hf[j] = 1 / h_theta^(2j/42) with h_theta = 1e4 * 4^(42/40) (NTK-scaled)."""
    dim_h = 42
    h_theta = 10000.0 * 4.0 ** (dim_h / (dim_h - 2))
    ex = (np.arange(21, dtype=np.float64) * 2 / dim_h).astype(np.float32).astype(np.float64)
    hf = (1.0 / np.power(h_theta, ex)).astype(np.float32).astype(np.float64)
    a = np.zeros((Hp, Wp, 64), np.float32)
    y = np.arange(Hp, dtype=np.float64)[:, None, None]
    x = np.arange(Wp, dtype=np.float64)[None, :, None]
    a[:, :, 22:43] = (y * hf).astype(np.float32)
    a[:, :, 43:64] = (x * hf).astype(np.float32)
    return a.reshape(Hp * Wp, 64)


def rope_table(angles: np.ndarray) -> np.ndarray:
    """cos block then sin block, flat [2*L*half]; sin offset L*half (app/models/common.js:3-12)."""
    a = np.asarray(angles, np.float64)
    return np.concatenate([np.cos(a).reshape(-1), np.sin(a).reshape(-1)]).astype(np.float32)


def dit_rope_table(Hp: int, Wp: int) -> np.ndarray:
    return rope_table(dit_rope_angles(Hp, Wp))


def _ptr(b):
    if b is None:
        return None
    if isinstance(b, DeviceBuffer):
        return b.ptr
    return int(b)
