"""GPU parity of the matrix-vector kernels of the router and shared expert (mv_q8, q8_repack,
mv_bf16, mv_f32; shaders/engine/mv.hlsl) through the gd C ABI, against the oracle's Q8_0
decode and float64 products. q8_repack is bit-exact; the products are within 2e-5 of
|W| |x| per output (fp32 accumulation), over staged (n cols <= 16384) and unstaged
activations, 1 and 2 rows per wave, the three activations and accumulate mode."""
import ctypes as C

import numpy as np
import pytest

from gyrodx import KERNEL_DIR, native

pytestmark = pytest.mark.gpu
TIMEOUT = 30000


@pytest.fixture(scope="module")
def ctx():
    L = native.lib()
    opts = native.Options(0, 0, 0, 32 << 20, 1024)
    h = C.c_void_p()
    native.check(L.gd_create(C.byref(opts), C.byref(h)), "gd_create")
    yield h
    native.check(L.gd_destroy(h, TIMEOUT), "gd_destroy")


class Run:
    """Host-visible buffers and one dispatch per call, waited on."""

    def __init__(self, ctx):
        self.ctx, self.bufs, self.pipes = ctx, [], {}

    def buffer(self, data: np.ndarray | None, nbytes: int | None = None):
        h, info = C.c_void_p(), native.BufferInfo()
        n = data.nbytes if data is not None else nbytes
        native.check(native.lib().gd_create_resource(self.ctx, n, 1, C.byref(h), C.byref(info)), "gd_create_resource")
        self.bufs.append((h, info, n))
        if data is not None:
            C.memmove(info.mapped, np.ascontiguousarray(data).ctypes.data, n)
        return info

    def read(self, info, dtype, count):
        return np.ctypeslib.as_array(C.cast(info.mapped, C.POINTER(C.c_uint8)), (count * np.dtype(dtype).itemsize,)
                                     ).copy().view(dtype)

    def dispatch(self, name, cst, gx, gy=1):
        L = native.lib()
        if name not in self.pipes:
            code = (KERNEL_DIR / f"{name}.co").read_bytes()
            p = C.c_void_p()
            native.check(L.gd_create_pipeline(self.ctx, code, len(code), C.byref(p)))
            self.pipes[name] = p
        arr = (C.c_uint32 * len(cst))(*cst)
        print(f"{name}: constants {list(cst)} grid ({gx}, {gy})", flush=True)
        native.check(L.gd_begin(self.ctx, TIMEOUT))
        native.check(L.gd_dispatch(self.ctx, self.pipes[name], arr, len(cst), gx, gy, 1))
        t = C.c_uint64()
        native.check(L.gd_submit(self.ctx, C.byref(t)))
        native.check(L.gd_wait_compute(self.ctx, t, TIMEOUT))

    def close(self):
        L = native.lib()
        for h, _, _ in self.bufs:
            native.check(L.gd_release_buffer(self.ctx, h, TIMEOUT))
        for p in self.pipes.values():
            native.check(L.gd_release_pipeline(self.ctx, p, TIMEOUT))


def q8_rows(rng, rows, cols):
    src = np.zeros((rows, cols // 32, 34), np.uint8)
    src[:, :, :2] = (rng.uniform(-0.02, 0.02, (rows, cols // 32, 1)).astype(np.float16)).view(np.uint8)
    src[:, :, 2:] = rng.integers(-128, 128, (rows, cols // 32, 32)).astype(np.int8).view(np.uint8)
    return src.reshape(-1)


def fbits(v):
    return int(np.array([v], np.float32).view(np.uint32)[0])


def expected(W, x, act, scale, y0):
    z = scale * (x.astype(np.float64) @ W.astype(np.float64).T)
    if act == 1:
        z = z / (1 + np.exp(-z))
    elif act == 2:
        z = 1 / (1 + np.exp(-z))
    if y0 is not None:
        z = z + y0
    bound = 2e-5 * np.abs(x.astype(np.float64)) @ np.abs(W.astype(np.float64)).T * max(abs(scale), 1.0) + 1e-6
    return z, bound


def mv_case(run, name, wbuf, W, row_bytes, rows, cols, n, act, scale, mode, rpw, rng):
    x = rng.standard_normal((n, cols)).astype(np.float32)
    y0 = rng.standard_normal((n, rows)).astype(np.float32)
    xb, yb = run.buffer(x), run.buffer(y0)
    run.dispatch(name, [wbuf.srv_index, 0, rows, cols, xb.uav_index, 0, cols, n, yb.uav_index, 0, rows, mode, act,
                        fbits(scale), row_bytes, rpw], (rows + 8 * rpw - 1) // (8 * rpw))
    y = run.read(yb, np.float32, n * rows).reshape(n, rows)
    ref, bound = expected(W, x, act, scale, y0 if mode else None)
    err = np.abs(y - ref)
    print(f"{name} rows={rows} cols={cols} n={n} act={act} mode={mode} rpw={rpw}: "
          f"max err/bound {float((err / bound).max()):.3f}", flush=True)
    assert (err <= bound).all(), (name, n, act, mode, rpw)


@pytest.mark.parametrize("rows,cols", [(300, 2560), (37, 1088)])
def test_q8_repack_and_mv_q8(ctx, oracle_mod, rows, cols):
    rng = np.random.default_rng(rows + cols)
    src = q8_rows(rng, rows, cols)
    run = Run(ctx)
    try:
        sb = run.buffer(src)
        row_bytes = cols + cols // 16
        pb = run.buffer(None, rows * row_bytes)
        blocks = rows * cols // 32
        groups = (blocks + 255) // 256
        run.dispatch("q8_repack", [sb.srv_index, 0, rows, cols, 0, 0, 0, 0, pb.uav_index, 0, 0, 0, 0, 0, row_bytes, 0],
                     min(groups, 65535), (groups + 65534) // 65535)
        packed = run.read(pb, np.uint8, rows * row_bytes).reshape(rows, row_bytes)
        np.testing.assert_array_equal(packed, oracle_mod.q8_repack(src, rows, cols))
        W = oracle_mod.q8_0_decode_rows(src, rows, cols)
        for n, act, scale, mode, rpw in ((1, 0, 1.0, 0, 1), (3, 1, 0.5, 1, 2), (8, 2, 1.0, 0, 1), (8, 0, 2.0, 1, 2)):
            mv_case(run, "mv_q8", pb, W, row_bytes, rows, cols, n, act, scale, mode, rpw, rng)
    finally:
        run.close()


@pytest.mark.parametrize("name", ["mv_bf16", "mv_f32"])
def test_mv_bf16_f32(ctx, name):
    rng = np.random.default_rng(7 if name == "mv_bf16" else 8)
    rows, cols = 260, 2560
    W = rng.standard_normal((rows, cols)).astype(np.float32)
    if name == "mv_bf16":
        bits = (W.view(np.uint32) >> 16).astype(np.uint16)
        W = (bits.astype(np.uint32) << 16).view(np.float32)
        data, row_bytes = bits, cols * 2
    else:
        data, row_bytes = W, cols * 4
    run = Run(ctx)
    try:
        wb = run.buffer(data)
        for n, act, scale, mode, rpw in ((1, 0, 1.0, 0, 1), (5, 1, 0.25, 1, 2), (8, 2, 1.0, 0, 1)):
            mv_case(run, name, wb, W, row_bytes, rows, cols, n, act, scale, mode, rpw, rng)
    finally:
        run.close()
