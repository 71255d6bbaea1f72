"""GPU test of the wave top-k routing primitive (route_fast.h) through moe_prefill_topk, called
through the gd C ABI on hand-made router logits.

Selection rule of src/engine.zig:670-687: the k largest logits (softmax is monotonic), ties to
the lower expert index. The logits here are drawn from a handful of values, so exact ties are
everywhere, including across the 8th/9th boundary; the expected ids are a stable argsort. The
weights are the softmax of the selected logits renormalised over them (src/engine.zig:527-540),
times the layer's expert-weights scale.
"""
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


def host_buffer(ctx, nbytes):
    h, info = C.c_void_p(), native.BufferInfo()
    native.check(native.lib().gd_create_resource(ctx, nbytes, 1, C.byref(h), C.byref(info)), "gd_create_resource")
    return h, info


def run_topk(ctx, logits: np.ndarray, scale: float):
    L = native.lib()
    n, NE = logits.shape
    code = (KERNEL_DIR / "moe_prefill_topk.co").read_bytes()
    pipe = C.c_void_p()
    native.check(L.gd_create_pipeline(ctx, code, len(code), C.byref(pipe)))
    bufs = [host_buffer(ctx, nbytes) for nbytes in (logits.nbytes, n * 32, n * 32)]
    (lh, li), (ih, ii), (wh, wi) = bufs
    try:
        C.memmove(li.mapped, np.ascontiguousarray(logits, np.float32).ctypes.data, logits.nbytes)
        sbits = int(np.array([scale], np.float32).view(np.uint32)[0])
        cst = (C.c_uint32 * 9)(li.uav_index, 0, NE, n, sbits, ii.uav_index, 0, wi.uav_index, 0)
        print(f"moe_prefill_topk: n={n} NE={NE} scale={scale}", flush=True)
        native.check(L.gd_begin(ctx, TIMEOUT))
        native.check(L.gd_dispatch(ctx, pipe, cst, 9, (n + 3) // 4, 1, 1))
        ticket = C.c_uint64()
        native.check(L.gd_submit(ctx, C.byref(ticket)))
        native.check(L.gd_wait_compute(ctx, ticket, TIMEOUT))
        ids = np.ctypeslib.as_array(C.cast(ii.mapped, C.POINTER(C.c_uint32)), (n, 8)).copy()
        wts = np.ctypeslib.as_array(C.cast(wi.mapped, C.POINTER(C.c_float)), (n, 8)).copy()
    finally:
        for h, _ in bufs:
            native.check(L.gd_release_buffer(ctx, h, TIMEOUT))
        native.check(L.gd_release_pipeline(ctx, pipe, TIMEOUT))
    return ids, wts


def expected(logits: np.ndarray, scale: float):
    order = np.argsort(-logits.astype(np.float64), axis=1, kind="stable")[:, :8]
    top = np.take_along_axis(logits.astype(np.float64), order, axis=1)
    w = np.exp(top - top[:, :1])
    w /= w.sum(axis=1, keepdims=True)
    if scale not in (0.0, 1.0):
        w *= scale
    return order.astype(np.uint32), w


@pytest.mark.parametrize("NE,values,scale", [(256, 7, 1.0), (256, 3, 2.5), (200, 5, 1.0), (64, 2, 1.0), (9, 2, 1.0),
                                             (256, 0, 1.0)])
def test_topk_ties_to_lower_index(ctx, NE, values, scale):
    rng = np.random.default_rng(NE * 31 + values)
    n = 1000
    if values:
        logits = (rng.integers(0, values, (n, NE)) * 0.375 - 1.0).astype(np.float32)
    else:
        logits = rng.standard_normal((n, NE)).astype(np.float32)
    ids, wts = run_topk(ctx, logits, scale)
    exp_ids, exp_w = expected(logits, scale)
    np.testing.assert_array_equal(ids, exp_ids)
    np.testing.assert_allclose(wts, exp_w, rtol=2e-6, atol=0)
