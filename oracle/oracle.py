"""ctypes binding of the CPU oracle (oracle/gyro_oracle.c). TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module, and
only as the checker or the timed CPU baseline. The product never routes through it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libgyro_oracle.so"
REF_PATH = HERE / "_ref" / "libtq_ref.so"
CODEBOOK = HERE.parent / "gyro-dx_amd" / "data" / "gyro_codebook.f16"

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        build()
    L = C.CDLL(str(LIB_PATH))
    f32p, u8p, u32p = C.POINTER(C.c_float), C.POINTER(C.c_uint8), C.POINTER(C.c_uint32)
    L.go_init.argtypes = [u8p, C.c_size_t]
    L.go_fp16_to_fp32.argtypes = [C.c_uint16]
    L.go_fp16_to_fp32.restype = C.c_float
    L.go_row_bytes.argtypes = [C.c_uint32, C.c_uint64]
    L.go_row_bytes.restype = C.c_uint64
    L.go_trellis_state.argtypes = [C.c_uint32, u8p, C.c_uint32]
    L.go_trellis_state.restype = C.c_uint32
    L.go_decode_row.argtypes = [C.c_uint32, C.c_int32, u8p, C.c_size_t, f32p, C.c_size_t]
    L.go_rotate.argtypes = [f32p, C.c_size_t, C.c_size_t, C.POINTER(C.c_int8)]
    L.go_unrotate.argtypes = [f32p, C.c_size_t, C.c_size_t, C.POINTER(C.c_int8)]
    L.go_rotate_f32signs.argtypes = [f32p, C.c_size_t, C.c_size_t, f32p]
    L.go_softmax.argtypes = [f32p, C.c_size_t]
    L.go_topk.argtypes = [f32p, C.c_size_t, u32p, f32p, C.c_size_t]
    L.go_dot_row.argtypes = [C.c_uint32, u8p, f32p, C.c_size_t]
    L.go_dot_row.restype = C.c_float
    L.go_decode_row_fast.argtypes = [C.c_uint32, u8p, f32p, C.c_size_t]
    L.go_moe_ffn.argtypes = [C.c_void_p, f32p, C.c_size_t, f32p, C.c_void_p, C.c_uint32]
    L.go_moe_dense_f64.argtypes = [C.c_void_p, f32p, C.c_size_t, u32p, f32p, C.POINTER(C.c_double)]
    L.go_router_f64.argtypes = [C.c_void_p, f32p, C.c_size_t, C.POINTER(C.c_double)]
    L.go_rms_norm.argtypes = [f32p, f32p, f32p, C.c_size_t, C.c_float]
    cb = np.frombuffer(CODEBOOK.read_bytes(), dtype=np.uint8)
    rc = L.go_init(cb.ctypes.data_as(u8p), cb.size)
    if rc != 0:
        raise RuntimeError(f"go_init failed: {rc}")
    _lib = L
    return L


def ref_lib():
    """The reference's vendored C decoder (third_party/agention-gyro), compiled from its own
    sources into oracle/_ref; None when it was not built."""
    if not REF_PATH.exists():
        return None
    L = C.CDLL(str(REF_PATH))
    L.tq_dequantize_row.argtypes = [C.c_int, C.c_void_p, C.POINTER(C.c_float), C.c_int64]
    L.tq_dequantize_row.restype = C.c_int
    L.tq_hadamard_rotate.argtypes = [C.POINTER(C.c_float), C.c_int64, C.c_int, C.POINTER(C.c_int8)]
    L.tq_hadamard_unrotate.argtypes = L.tq_hadamard_rotate.argtypes
    return L


def _p(a, t):
    return a.ctypes.data_as(C.POINTER(t))


def decode_row(type_id: int, src: np.ndarray, n: int, state_bits: int = 15):
    out = np.empty(n, dtype=np.float32)
    src = np.ascontiguousarray(src, dtype=np.uint8)
    rc = lib().go_decode_row(type_id, state_bits, _p(src, C.c_uint8), src.size, _p(out, C.c_float), n)
    return rc, out


def rotate(v: np.ndarray, block: int, signs_i8: np.ndarray | None, inverse: bool = False):
    v = np.ascontiguousarray(v, dtype=np.float32).copy()
    s = None if signs_i8 is None else _p(np.ascontiguousarray(signs_i8, dtype=np.int8), C.c_int8)
    fn = lib().go_unrotate if inverse else lib().go_rotate
    rc = fn(_p(v, C.c_float), v.size, block, s)
    return rc, v


def topk(values: np.ndarray, k: int):
    v = np.ascontiguousarray(values, dtype=np.float32)
    ids = np.empty(k, dtype=np.uint32)
    w = np.empty(k, dtype=np.float32)
    lib().go_topk(_p(v, C.c_float), v.size, _p(ids, C.c_uint32), _p(w, C.c_float), k)
    return ids, w


class _GoLayer(C.Structure):
    _fields_ = [
        ("E", C.c_uint32), ("F", C.c_uint32), ("n_expert", C.c_uint32), ("n_used", C.c_uint32),
        ("expert_weights_scale", C.c_float),
        ("router", C.c_void_p), ("router_bias", C.c_void_p),
        ("gate", C.c_void_p), ("up", C.c_void_p), ("down", C.c_void_p),
        ("gate_type", C.c_void_p), ("up_type", C.c_void_p), ("down_type", C.c_void_p),
        ("gate_signs", C.c_void_p), ("down_signs", C.c_void_p),
        ("SF", C.c_uint32),
        ("sh_gate", C.c_void_p), ("sh_up", C.c_void_p), ("sh_down", C.c_void_p),
        ("sh_gate_inp", C.c_void_p), ("sh_gate_const", C.c_float), ("sh_type", C.c_uint32),
    ]


class _GoTrace(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in
                ("logits", "route_ids", "route_w", "route_order", "order_start", "xh", "act",
                 "down", "moe_out")]


class OracleLayer:
    """Holds a synth.Layer in the oracle's struct form (keeps every buffer alive)."""

    def __init__(self, layer):
        self.layer = layer
        self._keep = []
        L = layer

        def ptr(a):
            if a is None:
                return None
            a = np.ascontiguousarray(a)
            self._keep.append(a)
            return a.ctypes.data

        def ptr_array(mats):
            arr = (C.c_void_p * len(mats))(*[ptr(m) for m in mats])
            self._keep.append(arr)
            return C.cast(arr, C.c_void_p).value

        s = _GoLayer()
        s.E, s.F, s.n_expert, s.n_used = L.E, L.F, L.n_expert, L.n_used
        s.expert_weights_scale = L.expert_weights_scale
        s.router = ptr(L.router)
        s.router_bias = ptr(L.router_bias)
        s.gate, s.up, s.down = ptr_array(L.gate), ptr_array(L.up), ptr_array(L.down)
        types = np.ascontiguousarray(L.types, dtype=np.uint32)
        s.gate_type = ptr(np.ascontiguousarray(types[:, 0]))
        s.up_type = ptr(np.ascontiguousarray(types[:, 1]))
        s.down_type = ptr(np.ascontiguousarray(types[:, 2]))
        s.gate_signs = ptr(L.gate_signs)
        s.down_signs = ptr(L.down_signs)
        s.SF = L.SF
        s.sh_gate, s.sh_up, s.sh_down = ptr(L.sh_gate), ptr(L.sh_up), ptr(L.sh_down)
        s.sh_gate_inp = ptr(L.sh_gate_inp)
        s.sh_gate_const = 1.0
        s.sh_type = getattr(L, "sh_type", 30)
        self.struct = s

    def forward(self, x: np.ndarray, threads: int | None = None, trace: bool = False):
        L = self.layer
        x = np.ascontiguousarray(x, dtype=np.float32)
        n = x.shape[0]
        out = np.empty((n, L.E), dtype=np.float32)
        tr = None
        bufs = {}
        if trace:
            bufs = dict(logits=np.empty((n, L.n_expert), np.float32),
                        route_ids=np.empty((n, L.n_used), np.uint32),
                        route_w=np.empty((n, L.n_used), np.float32),
                        route_order=np.empty(n * L.n_used, np.uint32),
                        order_start=np.empty(L.n_expert + 1, np.uint32),
                        xh=np.empty((n, L.E), np.float32),
                        act=np.empty((n * L.n_used, L.F), np.float32),
                        down=np.empty((n * L.n_used, L.E), np.float32),
                        moe_out=np.empty((n, L.E), np.float32))
            tr = _GoTrace(**{k: v.ctypes.data for k, v in bufs.items()})
        threads = threads or os.cpu_count() or 1
        rc = lib().go_moe_ffn(C.byref(self.struct), _p(x, C.c_float), n, _p(out, C.c_float),
                              C.byref(tr) if tr is not None else None, threads)
        if rc != 0:
            raise RuntimeError(f"go_moe_ffn failed: {rc}")
        return (out, bufs) if trace else out

    def dense_f64(self, x: np.ndarray, route_ids: np.ndarray, route_w: np.ndarray) -> np.ndarray:
        L = self.layer
        x = np.ascontiguousarray(x, dtype=np.float32)
        ids = np.ascontiguousarray(route_ids, dtype=np.uint32)
        w = np.ascontiguousarray(route_w, dtype=np.float32)
        out = np.empty((x.shape[0], L.E), dtype=np.float64)
        rc = lib().go_moe_dense_f64(C.byref(self.struct), _p(x, C.c_float), x.shape[0],
                                    _p(ids, C.c_uint32), _p(w, C.c_float), _p(out, C.c_double))
        if rc != 0:
            raise RuntimeError(f"go_moe_dense_f64 failed: {rc}")
        return out

    def router_f64(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty((x.shape[0], self.layer.n_expert), dtype=np.float64)
        lib().go_router_f64(C.byref(self.struct), _p(x, C.c_float), x.shape[0], _p(out, C.c_double))
        return out


def rms_norm(x: np.ndarray, w: np.ndarray | None, eps: float) -> np.ndarray:
    """go_rms_norm (src/kernels.zig:281-291) on each row of x."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows = x.reshape(-1, x.shape[-1])
    out = np.empty_like(rows)
    wp = None if w is None else _p(np.ascontiguousarray(w, dtype=np.float32), C.c_float)
    for i in range(rows.shape[0]):
        lib().go_rms_norm(_p(out[i], C.c_float), _p(rows[i], C.c_float), wp, rows.shape[1], eps)
    return out.reshape(x.shape)


def stack_forward(layers, x: np.ndarray, threads: int | None = None) -> np.ndarray:
    """The residual MoE stack x <- x + MoE_l(RMSNorm_l(x)) over synth layers (rmsNorm of
    src/kernels.zig:281-291, the MoE layer of src/engine.zig:520-687, a plain residual add)."""
    x = np.ascontiguousarray(x, dtype=np.float32).copy()
    for L in layers:
        h = rms_norm(x, L.norm_weight, L.norm_eps)
        x = x + OracleLayer(L).forward(h, threads=threads)
    return x


def rel_rms(ref, cand) -> float:
    """tests/parity.py:28-44 of the reference: sqrt(sum d^2 / sum ref^2)."""
    ref = np.asarray(ref, dtype=np.float64).ravel()
    cand = np.asarray(cand, dtype=np.float64).ravel()
    den = float(np.sum(ref * ref))
    num = float(np.sum((ref - cand) ** 2))
    return (num / den) ** 0.5 if den > 0 else num ** 0.5


def cosine(ref, cand) -> float:
    ref = np.asarray(ref, dtype=np.float64).ravel()
    cand = np.asarray(cand, dtype=np.float64).ravel()
    na, nb = float(np.dot(ref, ref)), float(np.dot(cand, cand))
    return float(np.dot(ref, cand)) / (na * nb) ** 0.5 if na > 0 and nb > 0 else 1.0


def q8_0_decode_rows(src: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """Q8_0 rows (34-byte blocks: binary16 scale d, 32 int8 quants q) to fp32, w = d * q
    (src/kernels.zig:107-120, decodeRow of type_q8_0)."""
    b = np.ascontiguousarray(src, np.uint8).reshape(rows, cols // 32, 34)
    d = b[:, :, :2].copy().view(np.float16).astype(np.float32)
    q = b[:, :, 2:].view(np.int8).astype(np.float32)
    return (d * q).reshape(rows, cols)


def q8_repack(src: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """The device layout of shaders/engine/mv.hlsl:94-119: per row the cols int8 quants, then the
    cols / 32 binary16 scales; row bytes cols + cols / 16."""
    b = np.ascontiguousarray(src, np.uint8).reshape(rows, cols // 32, 34)
    return np.concatenate([b[:, :, 2:].reshape(rows, cols), b[:, :, :2].reshape(rows, cols // 16)], axis=1)


def q8_repacked_decode(packed: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """fp32 weights of repacked Q8_0 rows (mv.hlsl:64-76: d of block c / 32 times the quant)."""
    p = np.ascontiguousarray(packed, np.uint8).reshape(rows, cols + cols // 16)
    q = p[:, :cols].view(np.int8).astype(np.float32)
    d = p[:, cols:].copy().view(np.float16).astype(np.float32)
    return q * np.repeat(d, 32, axis=1)
