"""ctypes binding of the C++ MoE layer engine (include/gyro_moe.h)."""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import BUILD_DIR, KERNEL_DIR

LIB_PATH = BUILD_DIR / "libgyro_moe.so"
PATH_REFERENCE, PATH_DECODE, PATH_PREFILL, PATH_GENERIC = 0, 1, 2, 3


class LayerDesc(C.Structure):
    _fields_ = [("E", C.c_uint32), ("F", C.c_uint32), ("n_expert", C.c_uint32), ("n_used", C.c_uint32),
                ("expert_weights_scale", C.c_float),
                ("router", C.c_void_p), ("router_bias", C.c_void_p), ("gate_signs", C.c_void_p),
                ("down_signs", C.c_void_p), ("gate", C.c_void_p), ("up", C.c_void_p), ("down", C.c_void_p),
                ("types", C.c_void_p), ("SF", C.c_uint32), ("sh_gate", C.c_void_p), ("sh_up", C.c_void_p),
                ("sh_down", C.c_void_p), ("sh_gate_inp", C.c_void_p), ("norm_weight", C.c_void_p),
                ("norm_eps", C.c_float), ("sh_type", C.c_uint32)]


# GGML type of a shared expert's matrices (src/kernels.zig:7-10) -> the engine's gm_layer_desc code.
SHARED_KIND = {30: 0, 8: 1, 0: 2}


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built; run gyro-dx_amd/build.py")
        L = C.CDLL(str(LIB_PATH))
        vp, u32, f32p = C.c_void_p, C.c_uint32, C.POINTER(C.c_float)
        L.gm_create.argtypes = [C.c_char_p, u32, u32, C.POINTER(vp)]
        L.gm_destroy.argtypes = [vp]
        L.gm_destroy.restype = None
        L.gm_last_error.argtypes = [vp]
        L.gm_last_error.restype = C.c_char_p
        L.gm_add_layer.argtypes = [vp, C.POINTER(LayerDesc), C.POINTER(u32)]
        L.gm_forward.argtypes = [vp, u32, u32, f32p, u32, f32p]
        L.gm_last_routes.argtypes = [vp, u32, C.POINTER(u32), f32p]
        L.gm_last_sort.argtypes = [vp, u32, C.POINTER(u32), C.POINTER(u32)]
        L.gm_dequant.argtypes = [vp, u32, u32, u32, u32, u32, f32p]
        L.gm_dequant_as.argtypes = [vp, u32, u32, u32, u32, u32, u32, f32p]
        L.gm_set_tokens.argtypes = [vp, f32p, u32]
        L.gm_run.argtypes = [vp, u32, u32, u32, u32, C.POINTER(u32), u32, C.POINTER(C.c_double),
                             C.POINTER(C.c_double)]
        L.gm_run_bracketed.argtypes = [vp, u32, u32, u32, u32, C.POINTER(u32), u32, u32, C.POINTER(C.c_double),
                                       C.POINTER(C.c_double), C.POINTER(C.c_double)]
        L.gm_read_outputs.argtypes = [vp, f32p, u32]
        L.gm_last_tiles.argtypes = [vp, u32, C.POINTER(u32), C.POINTER(u32)]
        L.gm_forward_stack.argtypes = [vp, C.POINTER(u32), u32, u32, f32p, u32, f32p]
        L.gm_run_stack.argtypes = [vp, u32, u32, u32, u32, C.POINTER(u32), u32, C.POINTER(C.c_double),
                                   C.POINTER(C.c_double)]
        L.gm_forward_decode_noalloc.argtypes = [vp, u32, vp, u32, vp, vp]
        _lib = L
    return _lib


def _f32p(a):
    return a.ctypes.data_as(C.POINTER(C.c_float))


class Engine:
    """The MoE layer engine on one GPU. Layers come from gyrodx.synth.Layer objects."""

    def __init__(self, max_tok: int = 64, adapter: int = 0, kernel_dir=KERNEL_DIR):
        self._h = C.c_void_p()
        rc = lib().gm_create(str(kernel_dir).encode(), adapter, max_tok, C.byref(self._h))
        if rc != 0:
            raise RuntimeError(f"gm_create failed ({rc})")
        self.max_tok = max_tok
        self.E = None

    def _check(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed ({rc}): {lib().gm_last_error(self._h).decode()}")

    def close(self):
        if self._h:
            lib().gm_destroy(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def add_layer(self, layer) -> int:
        keep = []

        def ptr(a):
            if a is None:
                return None
            a = np.ascontiguousarray(a)
            keep.append(a)
            return a.ctypes.data

        def ptrs(mats):
            arr = (C.c_void_p * len(mats))(*[ptr(m) for m in mats])
            keep.append(arr)
            return C.cast(arr, C.c_void_p).value

        d = LayerDesc(E=layer.E, F=layer.F, n_expert=layer.n_expert, n_used=layer.n_used,
                      expert_weights_scale=layer.expert_weights_scale,
                      router=ptr(np.asarray(layer.router, np.float32)),
                      router_bias=ptr(None if layer.router_bias is None else np.asarray(layer.router_bias, np.float32)),
                      gate_signs=ptr(layer.gate_signs), down_signs=ptr(layer.down_signs),
                      gate=ptrs(layer.gate), up=ptrs(layer.up), down=ptrs(layer.down),
                      types=ptr(np.ascontiguousarray(layer.types, np.uint32).reshape(-1)),
                      SF=layer.SF, sh_gate=ptr(layer.sh_gate), sh_up=ptr(layer.sh_up), sh_down=ptr(layer.sh_down),
                      sh_gate_inp=ptr(None if layer.sh_gate_inp is None else np.asarray(layer.sh_gate_inp, np.float32)),
                      norm_weight=ptr(None if layer.norm_weight is None else np.asarray(layer.norm_weight, np.float32)),
                      norm_eps=layer.norm_eps, sh_type=SHARED_KIND[getattr(layer, "sh_type", 30)] if layer.SF else 0)
        idx = C.c_uint32()
        self._check(lib().gm_add_layer(self._h, C.byref(d), C.byref(idx)), "gm_add_layer")
        self.E, self.U, self.n_expert = layer.E, layer.n_used, layer.n_expert
        return idx.value

    def forward(self, layer: int, x: np.ndarray, path: int = PATH_DECODE) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty_like(x)
        self._check(lib().gm_forward(self._h, layer, path, _f32p(x), x.shape[0], _f32p(out)), "gm_forward")
        return out

    def last_routes(self, n: int):
        ids = np.empty((n, self.U), np.uint32)
        w = np.empty((n, self.U), np.float32)
        self._check(lib().gm_last_routes(self._h, n, ids.ctypes.data_as(C.POINTER(C.c_uint32)), _f32p(w)),
                    "gm_last_routes")
        return ids, w

    def last_sort(self, n: int):
        """Counting sort of the last prefill forward: (route_order[n * n_used], order_start[n_expert + 1])."""
        order = np.empty(n * self.U, np.uint32)
        start = np.empty(self.n_expert + 1, np.uint32)
        p = lambda a: a.ctypes.data_as(C.POINTER(C.c_uint32))
        self._check(lib().gm_last_sort(self._h, n, p(order), p(start)), "gm_last_sort")
        return order, start

    def dequant(self, layer: int, expert: int, proj: int, row0: int, rows: int, cols: int,
                decoder: int = 0) -> np.ndarray:
        """Rows of one expert projection through a path's device decoder: 0 the decode kernels',
        1 the prefill GEMMs' (fp32 scale x codebook), 2 the prefill B operand (binary16)."""
        out = np.empty((rows, cols), np.float32)
        self._check(lib().gm_dequant_as(self._h, layer, expert, proj, row0, rows, decoder, _f32p(out)), "gm_dequant_as")
        return out

    def set_tokens(self, x: np.ndarray):
        x = np.ascontiguousarray(x, np.float32)
        self._check(lib().gm_set_tokens(self._h, _f32p(x), x.shape[0]), "gm_set_tokens")
        self.n_tokens = x.shape[0]

    def run(self, path: int, batch: int, calls: int, layers, bracket: int = 0, first: int = 0):
        """Processes `calls` calls of `batch` device-resident tokens from token `first`; returns
        (device ms, wall ms, mean duration in us of the bracketed kernel's launches)."""
        arr = (C.c_uint32 * len(layers))(*layers)
        dev, wall, br = C.c_double(), C.c_double(), C.c_double()
        self._check(lib().gm_run_bracketed(self._h, path, batch, calls, first, arr, len(layers), bracket,
                                           C.byref(dev), C.byref(wall), C.byref(br)), "gm_run")
        return dev.value, wall.value, br.value

    def last_tiles(self, max_tiles: int = 4096) -> np.ndarray:
        """Tile list of the last prefill call: [count, 4] u32 {expert, first row, rows, 0}."""
        buf = np.zeros((max_tiles, 4), np.uint32)
        cnt = C.c_uint32()
        self._check(lib().gm_last_tiles(self._h, max_tiles, buf.ctypes.data_as(C.POINTER(C.c_uint32)), C.byref(cnt)),
                    "gm_last_tiles")
        return buf[:cnt.value].copy()

    def forward_stack(self, layers, x: np.ndarray, path: int = PATH_DECODE) -> np.ndarray:
        """x <- x + MoE_l(RMSNorm_l(x)) over the given layer indices."""
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty_like(x)
        arr = (C.c_uint32 * len(layers))(*layers)
        self._check(lib().gm_forward_stack(self._h, arr, len(layers), path, _f32p(x), x.shape[0], _f32p(out)),
                    "gm_forward_stack")
        return out

    def run_stack(self, path: int, batch: int, calls: int, layers, first: int = 0):
        """Timed stack passes over device-resident tokens; returns (device ms, wall ms)."""
        arr = (C.c_uint32 * len(layers))(*layers)
        dev, wall = C.c_double(), C.c_double()
        self._check(lib().gm_run_stack(self._h, path, batch, calls, first, arr, len(layers), C.byref(dev),
                                       C.byref(wall)), "gm_run_stack")
        return dev.value, wall.value

    def forward_decode_noalloc(self, layer: int, x_ptr: int, n: int, out_ptr: int, stream: int = 0):
        """Decode-path forward of n <= 8 tokens between device buffers (addresses x_ptr, out_ptr),
        queued on the hipStream_t `stream` (0: the engine's compute stream); allocates nothing and
        does not wait."""
        self._check(lib().gm_forward_decode_noalloc(self._h, layer, x_ptr, n, out_ptr, stream or None),
                    "gm_forward_decode_noalloc")

    def read_outputs(self, n: int) -> np.ndarray:
        out = np.empty((n, self.E), np.float32)
        self._check(lib().gm_read_outputs(self._h, _f32p(out), n), "gm_read_outputs")
        return out
