"""numpy front end for the C oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg use this module as the checker. The product package
(decisive_amd) never imports it.

Every wrapper names the function of oracle.c it calls; oracle.c cites the
reference file:line each function restates.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

_lib = None


def build(force: bool = False) -> Path:
    """Compile liboracle.so with the committed Makefile."""
    if force or not LIB_PATH.exists():
        subprocess.run(["make", "-s", "-C", str(HERE), "-B" if force else "all"], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(LIB_PATH))
        _declare(_lib)
    return _lib


P = ctypes.c_void_p
SZ = ctypes.c_size_t
I = ctypes.c_int
F = ctypes.c_float


def _declare(L):
    sig = {
        "or_packed_size": (SZ, [SZ, SZ, I]),
        "or_pack_g64": (I, [P, SZ, SZ, I, P]),
        "or_unpack_g64": (I, [P, SZ, I, P]),
        "or_project": (I, [P, I, SZ, P, SZ, P]),
        "or_g32_size": (SZ, [SZ, SZ]),
        "or_pack_g32_f16": (I, [P, SZ, SZ, P]),
        "or_unpack_g32_f16": (I, [P, SZ, P]),
        "or_group_scale": (F, [P, SZ, I]),
        "or_group_codes": (None, [P, SZ, F, I, P]),
        "or_weight_quantize": (I, [P, SZ, SZ, I, P, P]),
        "or_act_quantize": (None, [P, SZ, SZ, I, P, P]),
        "or_grouped_gemm": (None, [P, P, SZ, P, P, SZ, SZ, I, P]),
        "or_grouped_gemm_affine": (None, [P, P, SZ, P, P, P, SZ, SZ, I, P]),
        "or_fit_mse": (F, [P, SZ, I, P]),
        "or_fit_affine": (None, [P, SZ, I, P, P, P]),
        "or_weight_quantize_fitted": (I, [P, SZ, SZ, I, I, P, P, P]),
        "or_fit_nf4": (F, [P, SZ, P]),
        "or_nf4_value": (F, [I]),
        "or_rows_decode": (None, [P, P, P, I, SZ, SZ, P]),
        "or_matrix_apply": (None, [P, SZ, P, P, SZ, SZ, I, I, P]),
        "or_panel_bytes": (SZ, [SZ, SZ, I]),
        "or_panel_pack": (None, [P, P, SZ, SZ, I, P, P]),
        "or_panel_apply_avx2": (I, [P, P, P, SZ, SZ, I, P, P, SZ, I, P]),
        "or_has_avx2": (I, []),
        "or_i8_quantize_rows": (None, [P, SZ, SZ, P, P, P]),
        "or_i8_gemm": (None, [P, P, SZ, P, P, SZ, SZ, I, P, P]),
        "or_i8_gemm_fused": (None, [P, P, SZ, P, P, P, P, SZ, SZ, P]),
        "or_q4_quantize_rows": (I, [P, SZ, SZ, P]),
        "or_q4_rows_codes": (None, [P, SZ, SZ, P]),
        "or_w4a16": (None, [P, SZ, SZ, P, SZ, P]),
        "or_layernorm": (None, [P, SZ, SZ, P, P, F]),
        "or_gelu": (None, [P, SZ]),
        "or_rmsnorm": (None, [P, SZ, SZ, P, F, I, P]),
        "or_silu_mul": (None, [P, P, SZ]),
        "or_softmax": (None, [P, SZ]),
        "or_mean_rows": (None, [P, SZ, SZ, P]),
        "or_attention": (None, [P, P, P, SZ, SZ, SZ, F, P]),
        "or_silu_requant": (None, [P, P, SZ, SZ, P, P]),
        "or_conv_silu": (None, [P, SZ, SZ, P, P]),
        "or_delta_scan": (None, [P, SZ, I, I, I, P, P, P, P, P]),
        "or_delta_gate": (None, [P, SZ, I, I, P, P, P]),
        "or_rope": (None, [P, SZ, I, I, P, P]),
        "or_attention_gqa": (None, [P, P, P, SZ, SZ, I, I, I, F, P]),
        "or_attention_gate": (None, [P, SZ, I, I, P, P]),
        "or_f32_to_bf16_n": (None, [P, SZ, P]),
        "or_f32_to_f16_n": (None, [P, SZ, P]),
        "or_f16_to_f32_n": (None, [P, SZ, P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


class OracleError(ValueError):
    pass


# ---- IEEE conversions ----------------------------------------------------

def f32_to_bf16(x) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().or_f32_to_bf16_n(_p(x), x.size, _p(out))
    return out


def bf16_to_f32(h) -> np.ndarray:
    h = _c(h, np.uint16)
    return (h.astype(np.uint32) << 16).view(np.float32)


def f32_to_f16_bits(x) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().or_f32_to_f16_n(_p(x), x.size, _p(out))
    return out


def f16_bits_to_f32(h) -> np.ndarray:
    h = _c(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().or_f16_to_f32_n(_p(h), h.size, _p(out))
    return out


# ---- wire layouts ----------------------------------------------------------

def packed_size(rows, cols, bits) -> int:
    return int(lib().or_packed_size(rows, cols, bits))


def pack_g64(bf16, rows, cols, bits) -> np.ndarray:
    """or_pack_g64: packed.rs:31-56."""
    bf16 = _c(bf16, np.uint16).reshape(-1)
    size = packed_size(rows, cols, bits)
    if not size or bf16.size != rows * cols:
        raise OracleError("invalid group-64 matrix shape")
    out = np.empty(size, np.uint8)
    rc = lib().or_pack_g64(_p(bf16), rows, cols, bits, _p(out))
    if rc == -2:
        raise OracleError("nonfinite packed weight")
    if rc:
        raise OracleError("invalid group-64 matrix shape")
    return out


def unpack_g64(packed, bits) -> np.ndarray:
    """or_unpack_g64: packed.rs:59-73."""
    packed = _c(packed, np.uint8).reshape(-1)
    stride = packed_size(1, 64, bits)
    if packed.size == 0 or not stride or packed.size % stride:
        raise OracleError("invalid packed rows")
    out = np.empty(packed.size // stride * 64, np.float32)
    rc = lib().or_unpack_g64(_p(packed), packed.size, bits, _p(out))
    if rc:
        raise OracleError("invalid packed scale" if rc == -3 else "invalid packed rows")
    return out


def project(packed, bits, cols, x, outputs) -> np.ndarray:
    """or_project: packed.rs:75-119."""
    packed = _c(packed, np.uint8).reshape(-1)
    x = _c(x, np.float32).reshape(-1)
    y = np.empty(outputs, np.float32)
    rc = lib().or_project(_p(packed), bits, cols, _p(x), outputs, _p(y))
    if rc:
        raise OracleError("invalid packed readout" if rc == -1 else "nonfinite readout activation")
    return y


def pack_g32_f16(w, rows, cols) -> np.ndarray:
    w = _c(w, np.float32).reshape(-1)
    size = int(lib().or_g32_size(rows, cols))
    if not size or w.size != rows * cols:
        raise OracleError("invalid group-32 matrix shape")
    out = np.empty(size, np.uint8)
    rc = lib().or_pack_g32_f16(_p(w), rows, cols, _p(out))
    if rc:
        raise OracleError("nonfinite weight" if rc == -2 else "invalid group-32 matrix shape")
    return out


def unpack_g32_f16(packed) -> np.ndarray:
    packed = _c(packed, np.uint8).reshape(-1)
    if packed.size == 0 or packed.size % 18:
        raise OracleError("invalid packed rows")
    out = np.empty(packed.size // 18 * 32, np.float32)
    rc = lib().or_unpack_g32_f16(_p(packed), packed.size, _p(out))
    if rc:
        raise OracleError("invalid packed scale")
    return out


# ---- grouped quantizers ------------------------------------------------------

def group_scale(x, bits) -> float:
    x = _c(x, np.float32).reshape(-1)
    return float(lib().or_group_scale(_p(x), x.size, bits))


def group_codes(x, scale, bits) -> np.ndarray:
    x = _c(x, np.float32).reshape(-1)
    out = np.empty(x.size, np.int8)
    lib().or_group_codes(_p(x), x.size, np.float32(scale), bits, _p(out))
    return out


def weight_quantize(bf16, n, k, bits):
    """or_weight_quantize: int8.rs:51-152 -> (codes [n, G*64] i8, scales [n, G] f32)."""
    bf16 = _c(bf16, np.uint16).reshape(-1)
    g = (k + 63) // 64
    codes = np.empty((n, g * 64), np.int8)
    scales = np.empty((n, g), np.float32)
    rc = lib().or_weight_quantize(_p(bf16), n, k, bits, _p(codes), _p(scales))
    if rc:
        raise OracleError("non-finite INT8 weight" if rc == -2 else "invalid INT8 matrix shape")
    return codes, scales


def act_quantize(x, m, k, bits=8):
    """or_act_quantize: int8.rs:178-202 -> (q [m, G*64] i8, s [m, G] f32)."""
    x = _c(x, np.float32).reshape(-1)
    g = (k + 63) // 64
    q = np.empty((m, g * 64), np.int8)
    s = np.empty((m, g), np.float32)
    if m:
        lib().or_act_quantize(_p(x), m, k, bits, _p(q), _p(s))
    return q, s


def grouped_gemm(qx, sx, m, qw, sw, n, k, fused=True) -> np.ndarray:
    """or_grouped_gemm: int8.rs:524-585 (fused) / :259-287 (unfused)."""
    y = np.empty((m, n), np.float32)
    if m and n:
        lib().or_grouped_gemm(_p(_c(qx, np.int8)), _p(_c(sx, np.float32)), m,
                              _p(_c(qw, np.int8)), _p(_c(sw, np.float32)), n, k,
                              1 if fused else 0, _p(y))
    return y


def grouped_gemm_affine(qx, sx, m, qw, sw, offsets, n, k, fused=True) -> np.ndarray:
    """or_grouped_gemm_affine: int8.rs:524-571 (fused) / :259-287 (scalar) with the offset term."""
    y = np.empty((m, n), np.float32)
    if m and n:
        lib().or_grouped_gemm_affine(_p(_c(qx, np.int8)), _p(_c(sx, np.float32)), m, _p(_c(qw, np.int8)),
                                     _p(_c(sw, np.float32)), _p(_c(offsets, np.float32)), n, k,
                                     1 if fused else 0, _p(y))
    return y


def fit_mse(x, avx2=True):
    """or_fit_mse: quantization.rs:25-71 over one group -> (codes, scale)."""
    x = _c(x, np.float32).reshape(-1)
    out = np.zeros(x.size, np.int8)
    s = lib().or_fit_mse(_p(x), x.size, 1 if avx2 else 0, _p(out))
    return out, np.float32(s)


def fit_affine(x, avx2=True):
    """or_fit_affine: quantization.rs:147-200 over one group -> (codes, scale, offset)."""
    x = _c(x, np.float32).reshape(-1)
    out = np.zeros(x.size, np.int8)
    s, o = np.zeros(1, np.float32), np.zeros(1, np.float32)
    lib().or_fit_affine(_p(x), x.size, 1 if avx2 else 0, _p(out), _p(s), _p(o))
    return out, s[0], o[0]


def fit_nf4(x):
    """or_fit_nf4: quantization.rs:260-302 over one group -> (codes, scale)."""
    x = _c(x, np.float32).reshape(-1)
    out = np.zeros(x.size, np.int8)
    s = lib().or_fit_nf4(_p(x), x.size, _p(out))
    return out, np.float32(s)


def nf4_table() -> np.ndarray:
    """quantization.rs:3-20, as the oracle holds it."""
    return np.array([lib().or_nf4_value(i) for i in range(16)], np.float32)


def rows_decode(codes, scales, offsets, nf4, rows, cols) -> np.ndarray:
    """or_rows_decode: quantized_rows.rs:89-110 append over Q4 rows."""
    y = np.empty((rows, cols), np.float32)
    off = None if offsets is None else _p(_c(offsets, np.float32))
    lib().or_rows_decode(_p(_c(codes, np.int8)), _p(_c(scales, np.float32)), off, 1 if nf4 else 0, rows, cols,
                         _p(y))
    return y


def weight_quantize_fitted(bf16, n, k, mode, avx2=True):
    """or_weight_quantize_fitted: int8.rs:86-117, mode "mse" or "affine", or
    quantized_rows.rs:56-66 "nf4" -> (codes [n x G*64], scales [n x G],
    offsets [n x G])."""
    bf16 = _c(bf16, np.uint16).reshape(-1)
    g = (k + 63) // 64
    codes = np.empty((n, g * 64), np.int8)
    scales = np.empty((n, g), np.float32)
    offsets = np.empty((n, g), np.float32)
    rc = lib().or_weight_quantize_fitted(_p(bf16), n, k, {"mse": 1, "affine": 2, "nf4": 3}[mode], 1 if avx2 else 0,
                                         _p(codes), _p(scales), _p(offsets))
    if rc:
        raise OracleError("non-finite INT8 weight")
    return codes, scales, offsets


def pack_wire_codes(codes, scales, n, k):
    """A fitted Q4 matrix (codes in [-8, 7], any scales) in the g64/f32 wire
    layout of packed.rs:3-56: per 64-run, (code + 8) nibbles, low nibble the
    even k, then the f32 LE scale. k % 64 == 0."""
    g = k // 64
    c = (np.asarray(codes, np.int16).reshape(n, g, 64) + 8).astype(np.uint8)
    wire = np.empty((n, g, 36), np.uint8)
    wire[..., :32] = c[..., 0::2] | (c[..., 1::2] << 4)
    wire[..., 32:] = np.asarray(scales, np.float32).reshape(n, g, 1).view(np.uint8)
    return wire.reshape(-1)


def matrix_apply(x, m, qw, sw, n, k, act_bits=8, fused=True) -> np.ndarray:
    """or_matrix_apply: int8.rs:166-176."""
    x = _c(x, np.float32).reshape(-1)
    y = np.empty((m, n), np.float32)
    if m and n:
        lib().or_matrix_apply(_p(x), m, _p(_c(qw, np.int8)), _p(_c(sw, np.float32)), n, k,
                              act_bits, 1 if fused else 0, _p(y))
    return y


def panel_pack(codes, scales, n, k, bits):
    codes = _c(codes, np.int8)
    scales = _c(scales, np.float32)
    g = (k + 63) // 64
    data = np.empty(int(lib().or_panel_bytes(n, k, bits)), np.uint8)
    ps = np.empty((n + 7) // 8 * g * 8, np.float32)
    lib().or_panel_pack(_p(codes), _p(scales), n, k, bits, _p(data), _p(ps))
    return data, ps


def has_avx2() -> bool:
    return bool(lib().or_has_avx2())


def panel_apply_avx2(data, ps, n, k, bits, qx, sx, m, threads=1, poffsets=None) -> np.ndarray:
    """or_panel_apply_avx2: int8.rs:229-256 + :404-585; poffsets (affine offsets
    in the panel scale layout, e.g. panel_pack(codes, offsets, ...)[1]) adds
    int8.rs:566-571."""
    y = np.empty((m, n), np.float32)
    off = None if poffsets is None else _p(_c(poffsets, np.float32))
    rc = lib().or_panel_apply_avx2(_p(data), _p(ps), off, n, k, bits, _p(_c(qx, np.int8)),
                                   _p(_c(sx, np.float32)), m, threads, _p(y))
    if rc:
        raise OracleError("AVX2/FMA unavailable")
    return y


# ---- per-row int8 ---------------------------------------------------------------

def i8_quantize_rows(x, rows, k):
    """or_i8_quantize_rows: webgpu/int8.rs:107-145 -> (q [rows,k], scale [rows], sum [rows])."""
    x = _c(x, np.float32).reshape(-1)
    q = np.empty((rows, k), np.int8)
    s = np.empty(rows, np.float32)
    sums = np.empty(rows, np.int32)
    lib().or_i8_quantize_rows(_p(x), rows, k, _p(q), _p(s), _p(sums))
    return q, s, sums


def i8_gemm(qa, sa, m, qw, sw, n, k, threads=1, raw=True, scaled=True):
    """or_i8_gemm: webgpu/int8.rs:147-242 -> (i32 [m,n] or None, f32 [m,n] or None)."""
    r = np.empty((m, n), np.int32) if raw else None
    y = np.empty((m, n), np.float32) if scaled else None
    lib().or_i8_gemm(_p(_c(qa, np.int8)), _p(_c(sa, np.float32)), m, _p(_c(qw, np.int8)),
                     _p(_c(sw, np.float32)), n, k, threads,
                     _p(r) if raw else None, _p(y) if scaled else None)
    return r, y


def i8_gemm_fused(qa, sa, m, qg, sg, qu, su, n, k):
    """or_i8_gemm_fused: webgpu/int8.rs:226-230 -> f32 [m, n] = silu(gate) * up."""
    y = np.empty((m, n), np.float32)
    lib().or_i8_gemm_fused(_p(_c(qa, np.int8)), _p(_c(sa, np.float32)), m, _p(_c(qg, np.int8)),
                           _p(_c(sg, np.float32)), _p(_c(qu, np.int8)), _p(_c(su, np.float32)), n, k, _p(y))
    return y


def q4_quantize_rows(x_f16_bits, rows, k) -> np.ndarray:
    """or_q4_quantize_rows: webgpu/q4.rs:48-73 -> uint32 [rows*(k/8) + 2*rows]."""
    out = np.empty(rows * (k // 8) + 2 * rows, np.uint32)
    rc = lib().or_q4_quantize_rows(_p(_c(x_f16_bits, np.uint16)), rows, k, _p(out))
    if rc:
        raise OracleError("Q4 reduction must be a multiple of eight, at most 32768")
    return out


def q4_rows_split(words, rows, k):
    """(codes int8 [rows, k], scales f32 [rows], sums i32 [rows]) of a q4 buffer."""
    words = _c(words, np.uint32)
    codes = np.empty((rows, k), np.int8)
    lib().or_q4_rows_codes(_p(words), rows, k, _p(codes))
    base = rows * (k // 8)
    return codes, words[base:base + rows].view(np.float32).copy(), words[base + rows:base + 2 * rows].view(np.int32).copy()


# ---- W4A16 closed form and epilogues --------------------------------------------

def w4a16(x_f16_bits, m, k, w_dequant, n) -> np.ndarray:
    y = np.empty((m, n), np.float64)
    lib().or_w4a16(_p(_c(x_f16_bits, np.uint16)), m, k, _p(_c(w_dequant, np.float32)), n, _p(y))
    return y


def layernorm(x, w, b, eps):
    x = np.array(x, np.float32, copy=True, order="C")
    rows, d = x.shape
    lib().or_layernorm(_p(x), rows, d, _p(_c(w, np.float32)), _p(_c(b, np.float32)), np.float32(eps))
    return x


def gelu(x):
    x = np.array(x, np.float32, copy=True, order="C")
    lib().or_gelu(_p(x), x.size)
    return x


def rmsnorm(x, w, eps, zero_centered=True):
    x = _c(x, np.float32)
    rows, d = x.shape
    y = np.empty_like(x)
    lib().or_rmsnorm(_p(x), rows, d, _p(_c(w, np.float32)), np.float32(eps),
                     1 if zero_centered else 0, _p(y))
    return y


def silu_mul(gate, up):
    g = np.array(gate, np.float32, copy=True, order="C")
    lib().or_silu_mul(_p(g), _p(_c(up, np.float32)), g.size)
    return g


def softmax(x):
    x = np.array(x, np.float32, copy=True, order="C")
    lib().or_softmax(_p(x), x.size)
    return x


def mean_rows(x):
    x = _c(x, np.float32)
    rows, d = x.shape
    out = np.empty(d, np.float32)
    lib().or_mean_rows(_p(x), rows, d, _p(out))
    return out


def attention(q, k, v, heads, scale):
    q, k, v = (_c(a, np.float32) for a in (q, k, v))
    seq, width = q.shape
    out = np.empty_like(q)
    lib().or_attention(_p(q), _p(k), _p(v), seq, heads, width // heads, np.float32(scale), _p(out))
    return out


def silu_requant(gate, up):
    gate = _c(gate, np.float32)
    up = _c(up, np.float32)
    m, n = gate.shape
    q = np.empty((m, n), np.int8)
    s = np.empty((m, n // 64), np.float32)
    lib().or_silu_requant(_p(gate), _p(up), m, n, _p(q), _p(s))
    return q, s


def nprocs_env_default() -> int:
    return max(1, min(16, os.cpu_count() or 1))


# ---- Pplx decoder layer ops (backbone.rs, cpu.rs) ----

def conv_silu(x, w):
    """cpu.rs:372-391 over a fresh sequence: x [n x width], w [4 x width]."""
    x = _c(x, np.float32)
    n, width = x.shape
    out = np.empty_like(x)
    lib().or_conv_silu(_p(x), n, width, _p(_c(w, np.float32)), _p(out))
    return out


def delta_scan(conv, lh, lk, ld, a, b, decay, dt):
    """backbone.rs:349-408 for every head: returns heads [lh x n x ld]."""
    conv = _c(conv, np.float32)
    n = conv.shape[0]
    out = np.empty((lh, n, ld), np.float32)
    lib().or_delta_scan(_p(conv), n, lh, lk, ld, _p(_c(a, np.float32)), _p(_c(b, np.float32)),
                        _p(_c(decay, np.float32)), _p(_c(dt, np.float32)), _p(out))
    return out


def delta_gate(heads, norm, z):
    """backbone.rs:310-326 + cpu.rs:392-414: heads [lh x n x ld], z [n x lh*ld]."""
    heads = _c(heads, np.float32)
    lh, n, ld = heads.shape
    out = np.empty((n, lh * ld), np.float32)
    lib().or_delta_gate(_p(heads), n, lh, ld, _p(_c(norm, np.float32)), _p(_c(z, np.float32)), _p(out))
    return out


def rope(x, heads, ad, positions, freq):
    """backbone.rs:415-428 on a copy of x [rows x heads*ad]."""
    x = np.array(x, np.float32, copy=True, order="C")
    pos = np.ascontiguousarray(positions, dtype=np.uint64)
    lib().or_rope(_p(x), x.shape[0], heads, ad, _p(pos), _p(_c(freq, np.float32)))
    return x


def attention_gqa(q, k, v, ah, akv, ad, scale):
    """backbone.rs:509-579 in f64: q [nq x ah*ad], k/v [nk x akv*ad] -> [ah x nq x ad]."""
    q, k, v = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32)
    nq, nk = q.shape[0], k.shape[0]
    out = np.empty((ah, nq, ad), np.float32)
    lib().or_attention_gqa(_p(q), _p(k), _p(v), nq, nk, ah, akv, ad, np.float32(scale), _p(out))
    return out


def attention_gate(heads, z):
    """cpu.rs:415-429: heads [ah x n x ad], z [n x ah*ad]."""
    heads = _c(heads, np.float32)
    ah, n, ad = heads.shape
    out = np.empty((n, ah * ad), np.float32)
    lib().or_attention_gate(_p(heads), n, ah, ad, _p(_c(z, np.float32)), _p(out))
    return out


def rope_freq():
    """backbone.rs:227-229: inv_freq[i] = 1 / 1e7^((2i)/64) in f32."""
    return np.array([np.float32(1.0) / np.power(np.float32(10_000_000.0), np.float32(2 * i) / np.float32(64.0),
                                                dtype=np.float32) for i in range(32)], np.float32)
