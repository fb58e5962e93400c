"""ctypes front end of libdecisive_rocm.so (the C ABI in include/decisive_rocm.h).

This is the Python-side binding a test or benchmark uses; the reference's Rust
host would bind the same symbols with `extern "C"`. Device buffers are passed
as integer addresses (torch tensors' data_ptr() work). There is no fallback:
when the shared library is missing or the GPU is not a gfx950, calls raise.
"""
from __future__ import annotations

import contextlib
import ctypes
import gc
import json
import re
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "lib" / "libdecisive_rocm.so"
HEADER = PKG.parent / "include" / "decisive_rocm.h"

# dz_status (src/inference/mod.rs:44-85 codes)
OK = 0
STATUS_NAMES = {
    0: "OK", 1: "INVALID_REQUEST", 2: "INVALID_PARAMETERS", 3: "CANCELLED", 4: "CACHE_OWNER",
    5: "INPUT_TOO_LONG", 6: "GPU_UNAVAILABLE", 7: "RESOURCE_LIMIT", 8: "MISSING_GPU_FEATURE",
    9: "INFERENCE_FAILED", 10: "INVALID_CHECKPOINT", 11: "UNSUPPORTED_CACHE",
}
Q4_G64_F32, Q8_G64_F32, Q4_G32_F16 = 0, 1, 2
F32, F16, BF16 = 0, 1, 2
EPI_NONE, EPI_GELU, EPI_RESIDUAL = 0, 1, 2
W4A8, W4A4, W4A16 = 0, 1, 2
PPLX_RESIDENT, PPLX_STREAMED = 0, 1
PPLX_WHOLE, PPLX_MIXER, PPLX_MLP = 0, 1, 2  # dz_pplx_layer_part's parts
FIT_SCALED, FIT_AFFINE, FIT_NF4 = 0, 1, 2  # dz_weight_upload_fitted's forms
ROWS_PACKED = -1  # dz_pplx_set_rows_form's default


class DzError(RuntimeError):
    """A non-OK dz_status; `code` is the reference's error-code string."""

    def __init__(self, status: int, message: str):
        self.status = status
        self.code = STATUS_NAMES.get(status, "UNKNOWN")
        super().__init__(f"{self.code}: {message}")


@contextlib.contextmanager
def capture(graph, stream):
    """`torch.cuda.graph(graph, stream=stream)` with Python's cyclic garbage
    collector held off while the graph records. The finalizers of `Weight` and
    `Context` free device memory (hipFree), and a free made while any stream
    records in the default (global) capture mode invalidates the recording. A
    collection pass can run at any allocation and finalize objects kept alive by
    reference cycles (an earlier exception's traceback, say), so one pass runs
    before the recording starts and none during it."""
    import torch

    gc.collect()
    enabled = gc.isenabled()
    gc.disable()
    try:
        with torch.cuda.graph(graph, stream=stream):
            yield
    finally:
        if enabled:
            gc.enable()


class EncoderConfig(ctypes.Structure):
    _fields_ = [("layers", ctypes.c_int32), ("hidden", ctypes.c_int32), ("heads", ctypes.c_int32),
                ("head_dim", ctypes.c_int32), ("ffn", ctypes.c_int32), ("vocab", ctypes.c_int32),
                ("ln_eps", ctypes.c_float)]


class PplxConfig(ctypes.Structure):
    _fields_ = [("layers", ctypes.c_int32), ("hidden", ctypes.c_int32), ("ff", ctypes.c_int32),
                ("delta_heads", ctypes.c_int32), ("delta_key_heads", ctypes.c_int32),
                ("delta_head_dim", ctypes.c_int32), ("attn_heads", ctypes.c_int32),
                ("attn_kv_heads", ctypes.c_int32), ("attn_head_dim", ctypes.c_int32)]


_lib = None

P, SZ, I32, U32, U64, F = (ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int32, ctypes.c_uint32,
                           ctypes.c_uint64, ctypes.c_float)
PP = ctypes.POINTER(ctypes.c_void_p)

_SIGNATURES = {
    "dz_status_name": (ctypes.c_char_p, [I32]),
    "dz_init": (I32, [I32, PP]),
    "dz_destroy": (None, [P]),
    "dz_last_error": (ctypes.c_char_p, [P]),
    "dz_set_stream": (I32, [P, P]),
    "dz_sync": (I32, [P]),
    "dz_capture_id": (I32, [P, ctypes.POINTER(ctypes.c_uint64)]),
    "dz_capture_release": (I32, [P, ctypes.c_uint64]),
    "dz_capture_release_all": (I32, [P]),
    "dz_info": (I32, [P, ctypes.c_char_p, SZ]),
    "dz_alloc": (I32, [P, SZ, PP]),
    "dz_free": (I32, [P, P]),
    "dz_copy_h2d": (I32, [P, P, P, SZ]),
    "dz_copy_d2h": (I32, [P, P, P, SZ]),
    "dz_weight_upload": (I32, [P, P, SZ, I32, SZ, SZ, PP]),
    "dz_weight_upload_fitted": (I32, [P, P, SZ, SZ, SZ, I32, P, PP]),
    "dz_weight_quantize": (I32, [P, P, I32, SZ, SZ, I32, I32, PP]),
    "dz_weight_free": (I32, [P, P]),
    "dz_weight_info": (I32, [P, ctypes.POINTER(SZ), ctypes.POINTER(SZ), ctypes.POINTER(I32),
                             ctypes.POINTER(I32), ctypes.POINTER(SZ)]),
    "dz_dequant": (I32, [P, P, P]),
    "dz_dequant_rows": (I32, [P, P, P, SZ, P, I32]),
    "dz_act_quantize": (I32, [P, P, SZ, SZ, I32, P, P]),
    "dz_linear": (I32, [P, P, P, I32, SZ, P, I32]),
    "dz_linear_noalloc": (I32, [P, P, P, I32, SZ, P, I32]),
    "dz_linear_pair": (I32, [P, P, P, P, SZ, P, P, I32]),
    "dz_linear_f16": (I32, [P, P, P, SZ, P, I32, P]),
    "dz_mlp_requant": (I32, [P, P, P, P, SZ, P, P]),
    "dz_linear_q8": (I32, [P, P, P, P, SZ, P]),
    "dz_project": (I32, [P, P, P, SZ, P]),
    "dz_act_quantize_records": (I32, [P, P, SZ, SZ, P]),
    "dz_linear_records": (I32, [P, P, P, SZ, P]),
    "dz_i8_quantize_rows": (I32, [P, P, SZ, SZ, P, P, P]),
    "dz_i8_gemm": (I32, [P, P, P, SZ, P, P, SZ, SZ, P, I32]),
    "dz_i8_gemm_fused": (I32, [P, P, P, SZ, P, P, P, P, SZ, SZ, P]),
    "dz_q4_quantize_rows": (I32, [P, P, I32, SZ, SZ, P]),
    "dz_q4_rows_gemm": (I32, [P, P, P, SZ, P, SZ, SZ, P, I32]),
    "dz_layernorm": (I32, [P, P, P, I32, SZ, SZ, P, P, F]),
    "dz_rmsnorm": (I32, [P, P, P, SZ, SZ, P, F, I32]),
    "dz_gelu": (I32, [P, P, I32, SZ]),
    "dz_silu_mul": (I32, [P, P, P, SZ]),
    "dz_add": (I32, [P, P, P, I32, SZ]),
    "dz_softmax_rows": (I32, [P, P, SZ, SZ]),
    "dz_mean_rows": (I32, [P, P, I32, SZ, SZ, SZ, P]),
    "dz_attention": (I32, [P, P, P, SZ, SZ, SZ, SZ, F]),
    "dz_encoder_create_random": (I32, [P, ctypes.POINTER(EncoderConfig), U64, PP]),
    "dz_encoder_destroy": (None, [P, P]),
    "dz_encoder_embedding_row_bytes": (I32, [P, ctypes.POINTER(SZ)]),
    "dz_encoder_read_rows": (I32, [P, P, P, SZ, P]),
    "dz_encoder_weight": (P, [P, I32, I32]),
    "dz_encoder_forward": (I32, [P, P, P, SZ, SZ, P]),
    "dz_encoder_forward_rows": (I32, [P, P, P, SZ, SZ, P]),
    "dz_encoder_hidden_rows": (I32, [P, P, P, SZ, P]),
    "dz_readout": (I32, [P, P, P, P, SZ, F, P]),
    "dz_encoder_readout_params": (I32, [P, PP, PP]),
    "dz_encoder_readout_rows": (I32, [P, P, P, SZ, P, SZ, P]),
    "dz_encoder_set_readout": (I32, [P, P, P, SZ, I32, P]),
    "dz_pplx_create": (I32, [P, ctypes.POINTER(PplxConfig), PP]),
    "dz_pplx_destroy": (None, [P, P]),
    "dz_pplx_set_weight": (I32, [P, P, ctypes.c_char_p, P, SZ, I32, SZ, SZ]),
    "dz_pplx_set_weight_fitted": (I32, [P, P, ctypes.c_char_p, P, SZ, SZ, SZ, I32]),
    "dz_pplx_set_rows_form": (I32, [P, P, I32]),
    "dz_pplx_set_vector": (I32, [P, P, ctypes.c_char_p, P, SZ]),
    "dz_pplx_layer": (I32, [P, P, I32, P, SZ, P, SZ]),
    "dz_pplx_layer_part": (I32, [P, P, I32, I32, P, SZ, P, SZ]),
    "dz_pplx_activation": (I32, [P, P, ctypes.c_char_p, P, SZ]),
    "dz_pplx_forward_rows": (I32, [P, P, P, SZ, P, SZ, P]),
    "dz_pplx_set_residency": (I32, [P, P, I32]),
    "dz_pplx_residency_info": (I32, [P, P, ctypes.c_char_p, SZ]),
    "dz_tune": (I32, [P, U32, ctypes.c_char_p, ctypes.c_char_p, SZ]),
    "dz_select_variant": (I32, [P, ctypes.c_char_p, ctypes.c_char_p]),
}


def header_symbols() -> list[str]:
    """Every function the C header declares."""
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(dz_[a-z0-9_]+)\s*\(", text)))


def load():
    """Loads the in-tree library; raises when it has not been built."""
    global _lib
    if _lib is None:
        try:
            # torch wheels bundle their own libamdhip64.so.7; loading torch first
            # makes this library bind to that same runtime (one HIP runtime per
            # process). Without torch the library uses /opt/rocm's runtime.
            import torch  # noqa: F401
        except ImportError:
            pass
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: run decisive_amd/build.py (no CPU fallback exists)")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def _addr(x) -> int | None:
    if x is None:
        return None
    if isinstance(x, int):
        return x
    if hasattr(x, "data_ptr"):
        return x.data_ptr()
    if hasattr(x, "ctypes"):
        return x.ctypes.data
    raise TypeError(f"cannot take the address of {type(x)}")


class Weight:
    """A device-resident quantized weight (dz_weight)."""

    def __init__(self, ctx: "Context", handle: int, owned: bool = True):
        self.ctx = ctx
        self.handle = handle
        self.owned = owned
        rows, cols, dbytes = SZ(), SZ(), SZ()
        bits, group = I32(), I32()
        load().dz_weight_info(handle, ctypes.byref(rows), ctypes.byref(cols), ctypes.byref(bits),
                              ctypes.byref(group), ctypes.byref(dbytes))
        self.rows, self.cols, self.bits, self.group = rows.value, cols.value, bits.value, group.value
        self.device_bytes = dbytes.value

    def free(self):
        if self.handle and self.owned:
            self.ctx._check(load().dz_weight_free(self.ctx.handle, self.handle))
        self.handle = 0

    def __del__(self):
        try:
            if self.handle and self.owned and self.ctx.handle:
                load().dz_weight_free(self.ctx.handle, self.handle)
                self.handle = 0
        except Exception:
            pass


class Context:
    """A dz_ctx on one HIP device."""

    def __init__(self, device: int = 0):
        L = load()
        h = ctypes.c_void_p()
        rc = L.dz_init(device, ctypes.byref(h))
        if rc != OK:
            raise DzError(rc, f"dz_init(device={device}) failed")
        self.handle = h.value
        self._keep = []

    def close(self):
        if self.handle:
            load().dz_destroy(self.handle)
            self.handle = 0

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc: int):
        if rc != OK:
            msg = load().dz_last_error(self.handle)
            raise DzError(rc, msg.decode() if msg else "")

    # ---- plumbing ----
    def set_stream(self, stream: int | None):
        self._check(load().dz_set_stream(self.handle, stream))

    def sync(self):
        self._check(load().dz_sync(self.handle))

    def info(self) -> dict:
        buf = ctypes.create_string_buffer(1 << 16)
        self._check(load().dz_info(self.handle, buf, len(buf)))
        return json.loads(buf.value.decode())

    def capture_id(self) -> int:
        """dz_capture_id: the id of the capture the context stream records."""
        out = ctypes.c_uint64()
        self._check(load().dz_capture_id(self.handle, ctypes.byref(out)))
        return out.value

    def capture_release(self, capture_id: int):
        """dz_capture_release: gives back what a destroyed graph's capture holds."""
        self._check(load().dz_capture_release(self.handle, capture_id))

    def capture_release_all(self):
        self._check(load().dz_capture_release_all(self.handle))

    # ---- weights ----
    def upload(self, packed, layout: int, rows: int, cols: int) -> Weight:
        import numpy as np
        packed = np.ascontiguousarray(packed, dtype=np.uint8)
        h = ctypes.c_void_p()
        self._check(load().dz_weight_upload(self.handle, packed.ctypes.data, packed.nbytes, layout, rows, cols,
                                            ctypes.byref(h)))
        return Weight(self, h.value)

    def upload_fitted(self, packed, rows: int, cols: int, form: int, offsets=None) -> Weight:
        """dz_weight_upload_fitted: a fitted Q4 g64/f32 wire matrix (full code range,
        signed scales) of `form` (FIT_SCALED, FIT_AFFINE with f32 offsets
        [rows x cols/64], FIT_NF4)."""
        import numpy as np
        packed = np.ascontiguousarray(packed, dtype=np.uint8)
        off = None if offsets is None else np.ascontiguousarray(offsets, dtype=np.float32)
        h = ctypes.c_void_p()
        self._check(load().dz_weight_upload_fitted(self.handle, packed.ctypes.data, packed.nbytes, rows, cols, form,
                                                   None if off is None else off.ctypes.data, ctypes.byref(h)))
        return Weight(self, h.value)

    def quantize(self, values, dtype: int, rows: int, cols: int, bits: int = 4, group: int = 64) -> Weight:
        h = ctypes.c_void_p()
        self._check(load().dz_weight_quantize(self.handle, _addr(values), dtype, rows, cols, bits, group,
                                              ctypes.byref(h)))
        return Weight(self, h.value)

    def dequant(self, w: Weight, y):
        self._check(load().dz_dequant(self.handle, w.handle, _addr(y)))

    def dequant_rows(self, w: Weight, ids, count: int, y, dtype: int = F32):
        self._check(load().dz_dequant_rows(self.handle, w.handle, _addr(ids), count, _addr(y), dtype))

    # ---- products ----
    def act_quantize(self, x, m: int, k: int, bits: int, q, s):
        self._check(load().dz_act_quantize(self.handle, _addr(x), m, k, bits, _addr(q), _addr(s)))

    def linear(self, w: Weight, x, x_dtype: int, m: int, y, mode: int):
        self._check(load().dz_linear(self.handle, w.handle, _addr(x), x_dtype, m, _addr(y), mode))

    def linear_noalloc(self, w: Weight, x, x_dtype: int, m: int, y, mode: int):
        self._check(load().dz_linear_noalloc(self.handle, w.handle, _addr(x), x_dtype, m, _addr(y), mode))

    def linear_f16(self, w: Weight, x, m: int, y, epilogue: int = 0, residual=None):
        self._check(load().dz_linear_f16(self.handle, w.handle, _addr(x), m, _addr(y), epilogue, _addr(residual)))

    def linear_pair(self, a: Weight, b: Weight, x, m: int, ya, yb, mode: int = W4A8):
        self._check(load().dz_linear_pair(self.handle, a.handle, b.handle, _addr(x), m, _addr(ya), _addr(yb), mode))

    def mlp_requant(self, gate: Weight, up: Weight, x, m: int, q, s):
        self._check(load().dz_mlp_requant(self.handle, gate.handle, up.handle, _addr(x), m, _addr(q), _addr(s)))

    def linear_q8(self, w: Weight, q, s, m: int, y):
        self._check(load().dz_linear_q8(self.handle, w.handle, _addr(q), _addr(s), m, _addr(y)))

    def project(self, w: Weight, x, m: int, y):
        self._check(load().dz_project(self.handle, w.handle, _addr(x), m, _addr(y)))

    def readout(self, w: Weight, norm, hidden, rows: int, eps: float, logits):
        self._check(load().dz_readout(self.handle, w.handle, _addr(norm), _addr(hidden), rows, eps,
                                      _addr(logits)))

    def act_quantize_records(self, x, m: int, k: int, records):
        self._check(load().dz_act_quantize_records(self.handle, _addr(x), m, k, _addr(records)))

    def linear_records(self, w: Weight, records, m: int, y):
        self._check(load().dz_linear_records(self.handle, w.handle, _addr(records), m, _addr(y)))

    def i8_quantize_rows(self, x, rows: int, k: int, q, scales, sums=None):
        self._check(load().dz_i8_quantize_rows(self.handle, _addr(x), rows, k, _addr(q), _addr(scales),
                                               _addr(sums)))

    def i8_gemm(self, a, sa, m: int, w, sw, n: int, k: int, y, raw: bool):
        self._check(load().dz_i8_gemm(self.handle, _addr(a), _addr(sa), m, _addr(w), _addr(sw), n, k, _addr(y),
                                      1 if raw else 0))

    def i8_gemm_fused(self, a, sa, m: int, wg, sg, wu, su, n: int, k: int, y):
        """silu(gate) * up of two per-row int8 products of the same codes
        (webgpu/int8.rs gemm(fused=true)); y f32 [m x n]."""
        self._check(load().dz_i8_gemm_fused(self.handle, _addr(a), _addr(sa), m, _addr(wg), _addr(sg), _addr(wu),
                                            _addr(su), n, k, _addr(y)))

    # ---- epilogues ----
    def q4_quantize_rows(self, values, dtype: int, rows: int, k: int, out):
        self._check(load().dz_q4_quantize_rows(self.handle, _addr(values), dtype, rows, k, _addr(out)))

    def q4_rows_gemm(self, a, sa, m: int, w, n: int, k: int, y, raw: bool):
        self._check(load().dz_q4_rows_gemm(self.handle, _addr(a), _addr(sa), m, _addr(w), n, k, _addr(y),
                                           1 if raw else 0))

    def layernorm(self, x, y, dtype: int, rows: int, d: int, w, b, eps: float):
        self._check(load().dz_layernorm(self.handle, _addr(x), _addr(y), dtype, rows, d, _addr(w), _addr(b), eps))

    def rmsnorm(self, x, y, rows: int, d: int, w, eps: float, zero_centered: bool = True):
        self._check(load().dz_rmsnorm(self.handle, _addr(x), _addr(y), rows, d, _addr(w), eps,
                                      1 if zero_centered else 0))

    def gelu(self, x, dtype: int, n: int):
        self._check(load().dz_gelu(self.handle, _addr(x), dtype, n))

    def silu_mul(self, g, u, n: int):
        self._check(load().dz_silu_mul(self.handle, _addr(g), _addr(u), n))

    def add(self, x, y, dtype: int, n: int):
        self._check(load().dz_add(self.handle, _addr(x), _addr(y), dtype, n))

    def softmax_rows(self, x, rows: int, n: int):
        self._check(load().dz_softmax_rows(self.handle, _addr(x), rows, n))

    def mean_rows(self, x, dtype: int, batch: int, rows: int, d: int, out):
        self._check(load().dz_mean_rows(self.handle, _addr(x), dtype, batch, rows, d, _addr(out)))

    def attention(self, qkv, out, batch: int, seq: int, heads: int, dh: int, scale: float):
        self._check(load().dz_attention(self.handle, _addr(qkv), _addr(out), batch, seq, heads, dh, scale))

    # ---- encoder ----
    def encoder_random(self, cfg: EncoderConfig, seed: int) -> "Encoder":
        h = ctypes.c_void_p()
        self._check(load().dz_encoder_create_random(self.handle, ctypes.byref(cfg), seed, ctypes.byref(h)))
        return Encoder(self, h.value, cfg)

    # ---- the Pplx decider ----
    def pplx_create(self, cfg: PplxConfig) -> "Pplx":
        h = ctypes.c_void_p()
        self._check(load().dz_pplx_create(self.handle, ctypes.byref(cfg), ctypes.byref(h)))
        return Pplx(self, h.value, cfg)

    # ---- tuner ----
    def tune(self, budget_ms: int, cache: str | None = None) -> dict:
        out = ctypes.create_string_buffer(1 << 16)
        self._check(load().dz_tune(self.handle, budget_ms, cache.encode() if cache else None, out, len(out)))
        return json.loads(out.value.decode())

    def select_variant(self, family: str, name: str):
        self._check(load().dz_select_variant(self.handle, family.encode(), name.encode()))


class Encoder:
    """dz_encoder: the configuration-3 encoder with device-resident weights."""

    QKV, O, UP, DOWN, EMBED, READOUT = 0, 1, 2, 3, 4, 5
    READOUT_CODES = 255

    def __init__(self, ctx: Context, handle: int, cfg: EncoderConfig):
        self.ctx, self.handle, self.cfg = ctx, handle, cfg
        rb = SZ()
        ctx._check(load().dz_encoder_embedding_row_bytes(handle, ctypes.byref(rb)))
        self.row_bytes = rb.value

    def weight(self, layer: int, which: int) -> Weight:
        h = load().dz_encoder_weight(self.handle, layer, which)
        if not h:
            raise DzError(2, "no such encoder weight")
        return Weight(self.ctx, h, owned=False)

    def read_rows(self, ids):
        import numpy as np
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        out = np.empty(ids.size * self.row_bytes, np.uint8)
        self.ctx._check(load().dz_encoder_read_rows(self.ctx.handle, self.handle, ids.ctypes.data, ids.size,
                                                    out.ctypes.data))
        return out

    def forward(self, ids_dev, batch: int, seq: int, out):
        self.ctx._check(load().dz_encoder_forward(self.ctx.handle, self.handle, _addr(ids_dev), batch, seq, _addr(out)))

    def forward_rows(self, rows_host, batch: int, seq: int, out):
        import numpy as np
        rows_host = np.ascontiguousarray(rows_host, dtype=np.uint8)
        self.ctx._check(load().dz_encoder_forward_rows(self.ctx.handle, self.handle, rows_host.ctypes.data, batch,
                                                       seq, _addr(out)))

    def hidden_rows(self, rows_host, seq: int, hidden):
        import numpy as np
        rows_host = np.ascontiguousarray(rows_host, dtype=np.uint8)
        self.ctx._check(load().dz_encoder_hidden_rows(self.ctx.handle, self.handle, rows_host.ctypes.data, seq,
                                                      _addr(hidden)))

    def readout_params(self):
        """(readout Weight, device address of its norm weights)."""
        w, norm = ctypes.c_void_p(), ctypes.c_void_p()
        self.ctx._check(load().dz_encoder_readout_params(self.handle, ctypes.byref(w), ctypes.byref(norm)))
        return Weight(self.ctx, w.value, owned=False), norm.value

    def set_readout(self, packed_host, layout: int, norm_host):
        import numpy as np
        packed_host = np.ascontiguousarray(packed_host, dtype=np.uint8)
        norm_host = np.ascontiguousarray(norm_host, dtype=np.float32)
        self.ctx._check(load().dz_encoder_set_readout(self.ctx.handle, self.handle, packed_host.ctypes.data,
                                                      packed_host.size, layout, norm_host.ctypes.data))

    def readout_rows(self, rows_host, seq: int, markers):
        """Logits f32 [len(markers) x 255] of the hidden rows at markers."""
        import numpy as np
        rows_host = np.ascontiguousarray(rows_host, dtype=np.uint8)
        markers = np.ascontiguousarray(markers, dtype=np.int32)
        out = np.empty((markers.size, self.READOUT_CODES), np.float32)
        self.ctx._check(load().dz_encoder_readout_rows(self.ctx.handle, self.handle, rows_host.ctypes.data, seq,
                                                       markers.ctypes.data, markers.size, out.ctypes.data))
        return out

    def close(self):
        if self.handle:
            load().dz_encoder_destroy(self.ctx.handle, self.handle)
            self.handle = 0


class Pplx:
    """dz_pplx: the Pplx decider (hybrid gated-delta / attention decoder)."""

    def __init__(self, ctx: Context, handle: int, cfg: PplxConfig):
        self.ctx, self.handle, self.cfg = ctx, handle, cfg

    def set_weight(self, name: str, packed, layout: int, rows: int, cols: int):
        import numpy as np
        packed = np.ascontiguousarray(packed, dtype=np.uint8)
        self.ctx._check(load().dz_pplx_set_weight(self.ctx.handle, self.handle, name.encode(), packed.ctypes.data,
                                                  packed.size, layout, rows, cols))

    def set_weight_fitted(self, name: str, packed, rows: int, cols: int, form: int = FIT_SCALED):
        """dz_pplx_set_weight_fitted: a fitted Q4 g64/f32 wire projection (MSE form)."""
        import numpy as np
        packed = np.ascontiguousarray(packed, dtype=np.uint8)
        self.ctx._check(load().dz_pplx_set_weight_fitted(self.ctx.handle, self.handle, name.encode(),
                                                         packed.ctypes.data, packed.size, rows, cols, form))

    def set_rows_form(self, form: int):
        """dz_pplx_set_rows_form: ROWS_PACKED, FIT_SCALED or FIT_NF4 embedding rows."""
        self.ctx._check(load().dz_pplx_set_rows_form(self.ctx.handle, self.handle, form))

    def set_vector(self, name: str, values):
        import numpy as np
        values = np.ascontiguousarray(values, dtype=np.float32).ravel()
        self.ctx._check(load().dz_pplx_set_vector(self.ctx.handle, self.handle, name.encode(), values.ctypes.data,
                                                  values.size))

    def layer(self, index: int, hidden_dev, n: int, markers=None):
        import numpy as np
        m = None if markers is None else np.ascontiguousarray(markers, dtype=np.int32)
        self.ctx._check(load().dz_pplx_layer(self.ctx.handle, self.handle, index, _addr(hidden_dev), n,
                                             None if m is None else m.ctypes.data, 0 if m is None else m.size))

    def layer_part(self, index: int, part: int, hidden_dev, n: int, markers=None):
        """dz_pplx_layer_part: PPLX_MIXER or PPLX_MLP half of layer `index` in place."""
        import numpy as np
        m = None if markers is None else np.ascontiguousarray(markers, dtype=np.int32)
        self.ctx._check(load().dz_pplx_layer_part(self.ctx.handle, self.handle, index, part, _addr(hidden_dev), n,
                                                  None if m is None else m.ctypes.data, 0 if m is None else m.size))

    def activation(self, name: str, out_dev):
        """dz_pplx_activation: the last layer call's activation `name` into out_dev (a device tensor of
        exactly its size)."""
        nbytes = out_dev.numel() * out_dev.element_size()
        self.ctx._check(load().dz_pplx_activation(self.ctx.handle, self.handle, name.encode(), _addr(out_dev),
                                                  nbytes))

    def forward_rows(self, rows_host, n: int, markers):
        """Logits f32 [len(markers) x 255]."""
        import numpy as np
        rows_host = np.ascontiguousarray(rows_host, dtype=np.uint8)
        m = np.ascontiguousarray(markers, dtype=np.int32)
        out = np.empty((m.size, 255), np.float32)
        self.ctx._check(load().dz_pplx_forward_rows(self.ctx.handle, self.handle, rows_host.ctypes.data, n,
                                                    m.ctypes.data, m.size, out.ctypes.data))
        return out

    def set_residency(self, residency: int):
        """PPLX_RESIDENT or PPLX_STREAMED (two device banks, layers copied in turn)."""
        self.ctx._check(load().dz_pplx_set_residency(self.ctx.handle, self.handle, residency))

    def residency_info(self) -> dict:
        buf = ctypes.create_string_buffer(1024)
        self.ctx._check(load().dz_pplx_residency_info(self.ctx.handle, self.handle, buf, len(buf)))
        return json.loads(buf.value.decode())

    def close(self):
        if self.handle:
            load().dz_pplx_destroy(self.ctx.handle, self.handle)
            self.handle = 0
