"""GPU tests of the gyro_native C ABI on MI355X, called through ctypes.

Mirrors the reference's hardware conformance commands (src/native.zig): `gyro` (the scalar
decoder bit-identical to the CPU for all 8 types, :119-152), `linalg` (one exact 16x16x16 matrix
product, native/gyro_native.cpp:532-595) and `stream` (file ranges into a buffer read back
equal, :72-117), plus the dispatch contract of native/gyro_native.cpp:874-951.
"""
import ctypes as C
import os
import tempfile

import numpy as np
import pytest

from gyrodx import CODEBOOK, KERNEL_DIR, native

pytestmark = pytest.mark.gpu
TIMEOUT = 30000
TYPES = [(144, 34), (145, 26), (146, 30), (147, 42), (148, 50), (149, 58), (150, 22), (151, 18)]
EDGE_SCALES = [0x0000, 0x8000, 0x0001, 0x8001, 0x03FF, 0x83FF, 0x0400, 0x8400, 0x3C00, 0xBC00, 0x7BFF, 0xFBFF]


@pytest.fixture(scope="module")
def ctx():
    L = native.lib()
    opts = native.Options(0, 0, 0, 32 << 20, 1024)
    h = C.c_void_p()
    native.check(L.gd_create(C.byref(opts), C.byref(h)), "gd_create")
    yield h
    native.check(L.gd_destroy(h, TIMEOUT), "gd_destroy")


def code(name):
    return (KERNEL_DIR / f"{name}.co").read_bytes()


def test_caps(ctx):
    caps = native.Caps()
    native.check(native.lib().gd_get_caps(ctx, C.byref(caps)))
    assert caps.vendor_id == 0x1002
    assert caps.shader_model >= 0x66  # src/gpu.zig:48
    assert caps.abi_version == 1
    assert caps.dedicated_video_bytes > 100 << 30
    print("adapter", caps.adapter_name.decode(), hex(caps.device_id))


def test_validate_gyro_reference_recipe(ctx, oracle_mod):
    """src/native.zig:119-152: LCG bytes, 12 edge scales, 64 blocks per type, bit-exact."""
    L = native.lib()
    dec = code("gyro_decode")
    book = CODEBOOK.read_bytes()
    state = 0x4759524F
    for type_id, bb in TYPES:
        enc = bytearray(bb * 64)
        for i in range(len(enc)):
            state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
            enc[i] = state >> 24
        for block in range(64):
            s = EDGE_SCALES[block % len(EDGE_SCALES)]
            enc[block * bb] = s & 0xFF
            enc[block * bb + 1] = s >> 8
        enc = np.frombuffer(bytes(enc), np.uint8)
        rc, expected = oracle_mod.decode_row(type_id, enc, 128 * 64)
        assert rc == 0
        err = C.c_float()
        r = L.gd_validate_gyro(ctx, dec, len(dec), book, len(book), enc.ctypes.data, enc.size, type_id,
                               expected.ctypes.data, expected.size, C.byref(err), TIMEOUT)
        assert r == 0, (type_id, native.hresult(r), err.value)
        assert err.value == 0.0
        # A single flipped bit in the expected values must be reported.
        bad = expected.copy()
        bad.view(np.uint32)[77] ^= 1
        r = L.gd_validate_gyro(ctx, dec, len(dec), book, len(book), enc.ctypes.data, enc.size, type_id,
                               bad.ctypes.data, bad.size, C.byref(err), TIMEOUT)
        assert r == native.ERROR_INVALID_DATA


def test_validate_gyro_golden_fixture(ctx):
    """All 512 blocks of the independent C oracle fixture (tests/gyro_vectors.zig:28-60)."""
    from test_oracle_format import parse_fixture
    L = native.lib()
    dec = code("gyro_decode")
    book = CODEBOOK.read_bytes()
    cases, _ = parse_fixture()
    by_type = {}
    for type_id, enc, bits in cases:
        e, b = by_type.setdefault(type_id, (bytearray(), []))
        e += enc
        b.append(bits)
    for type_id, (enc, bits) in by_type.items():
        expected = np.concatenate(bits).view(np.float32)
        err = C.c_float()
        r = L.gd_validate_gyro(ctx, dec, len(dec), book, len(book), bytes(enc), len(enc), type_id,
                               expected.ctypes.data, expected.size, C.byref(err), TIMEOUT)
        assert r == 0, (type_id, native.hresult(r))


def test_validate_gyro_rejects_bad_arguments(ctx):
    L = native.lib()
    dec = code("gyro_decode")
    book = CODEBOOK.read_bytes()
    exp = np.zeros(128, np.float32)
    err = C.c_float()
    enc = bytes(34)
    assert L.gd_validate_gyro(ctx, dec, len(dec), book, 8191, enc, 34, 144, exp.ctypes.data, 128, C.byref(err), TIMEOUT) == native.E_INVALIDARG
    assert L.gd_validate_gyro(ctx, dec, len(dec), book, 8192, enc, 33, 144, exp.ctypes.data, 128, C.byref(err), TIMEOUT) == native.E_INVALIDARG
    assert L.gd_validate_gyro(ctx, dec, len(dec), book, 8192, enc, 34, 152, exp.ctypes.data, 128, C.byref(err), TIMEOUT) == native.E_INVALIDARG
    exp[3] = np.inf
    assert L.gd_validate_gyro(ctx, dec, len(dec), book, 8192, enc, 34, 144, exp.ctypes.data, 128, C.byref(err), TIMEOUT) == native.E_INVALIDARG


def test_validate_linalg(ctx):
    L = native.lib()
    smoke = code("linalg_smoke")
    err = C.c_float(-1)
    r = L.gd_validate_linalg(ctx, smoke, len(smoke), C.byref(err), TIMEOUT)
    assert r == 0, native.hresult(r)
    assert err.value == 0.0


def make_resource(ctx, nbytes, kind):
    h = C.c_void_p()
    info = native.BufferInfo()
    native.check(native.lib().gd_create_resource(ctx, nbytes, kind, C.byref(h), C.byref(info)), "gd_create_resource")
    return h, info


def test_dispatch_contract(ctx):
    """Host and device resources, the bit-exact copy, tickets, timestamps and argument checks."""
    L = native.lib()
    pipe = C.c_void_p()
    ew = code("ew")
    native.check(L.gd_create_pipeline(ctx, ew, len(ew), C.byref(pipe)))
    host, hinfo = make_resource(ctx, 4096, 1)
    dev, dinfo = make_resource(ctx, 4096, 0)
    assert hinfo.mapped and hinfo.allocated_bytes == 4096 and hinfo.srv_index != hinfo.uav_index
    assert not dinfo.mapped and dinfo.gpu_address
    src = (np.arange(1024, dtype=np.uint64) * 2654435761 % (1 << 32)).astype(np.uint32)
    C.memmove(hinfo.mapped, src.ctypes.data, 4096)
    assert L.gd_dispatch(ctx, pipe, None, 0, 1, 1, 1) == native.E_INVALIDARG  # not recording
    native.check(L.gd_begin(ctx, TIMEOUT))
    assert L.gd_begin(ctx, TIMEOUT) == native.E_ILLEGAL_METHOD_CALL  # no nesting
    ts0 = C.c_uint32()
    native.check(L.gd_timestamp(ctx, C.byref(ts0)))
    cst = (C.c_uint32 * 12)(hinfo.uav_index, 0, 0, hinfo.uav_index, 0, 0, dinfo.uav_index, 0, 0, 1024, 1, 5)
    native.check(L.gd_dispatch(ctx, pipe, cst, 12, 4, 1, 1))
    assert L.gd_dispatch(ctx, pipe, cst, 61, 4, 1, 1) == native.E_INVALIDARG
    assert L.gd_dispatch(ctx, pipe, cst, 12, 0, 1, 1) == native.E_INVALIDARG
    assert L.gd_dispatch(ctx, pipe, cst, 12, 65536, 1, 1) == native.E_INVALIDARG
    native.check(L.gd_barrier(ctx))
    ts1 = C.c_uint32()
    native.check(L.gd_timestamp(ctx, C.byref(ts1)))
    ticket = C.c_uint64()
    native.check(L.gd_submit(ctx, C.byref(ticket)))
    assert ticket.value >= 1
    native.check(L.gd_wait_compute(ctx, ticket, TIMEOUT))
    assert L.gd_wait_compute(ctx, ticket.value + 5, TIMEOUT) == native.E_INVALIDARG
    ticks = (C.c_uint64 * 2)()
    freq = C.c_uint64()
    native.check(L.gd_read_timestamps(ctx, 2, ticks, C.byref(freq)))
    assert freq.value == 1_000_000_000 and ticks[1] >= ticks[0]
    back = np.zeros(1024, np.uint32)
    native.check(L.gd_readback(ctx, dev, 0, 4096, back.ctypes.data, TIMEOUT))
    np.testing.assert_array_equal(back, src)
    s, c = C.c_uint64(), C.c_uint64()
    native.check(L.gd_poll(ctx, C.byref(s), C.byref(c)))
    assert c.value >= ticket.value
    native.check(L.gd_release_buffer(ctx, dev, TIMEOUT))
    native.check(L.gd_release_buffer(ctx, host, TIMEOUT))
    native.check(L.gd_release_pipeline(ctx, pipe, TIMEOUT))


def test_stream_file_ranges(ctx):
    """src/native.zig:72-117: raw ranges of a file land in a buffer and read back equal."""
    L = native.lib()
    data = np.random.default_rng(9).integers(0, 256, 1 << 20, dtype=np.uint8)
    with tempfile.NamedTemporaryFile(delete=False) as f:
        f.write(data.tobytes())
        path = f.name
    try:
        fh = C.c_void_p()
        native.check(L.gd_open_file(ctx, path.encode(), C.byref(fh)))
        size = C.c_uint64()
        native.check(L.gd_file_size(fh, C.byref(size)))
        assert size.value == data.size
        buf = C.c_void_p()
        native.check(L.gd_create_buffer(ctx, 300000, C.byref(buf)))
        ranges = (native.Range * 3)(native.Range(1000, 0, 100000, 0), native.Range(500000, 100000, 150000, 0),
                                    native.Range(7, 250000, 50000, 0))
        ticket = C.c_uint64()
        native.check(L.gd_read_ranges(ctx, fh, buf, ranges, 3, C.byref(ticket)))
        native.check(L.gd_wait_storage(ctx, ticket, TIMEOUT))
        back = np.zeros(300000, np.uint8)
        native.check(L.gd_readback(ctx, buf, 0, 300000, back.ctypes.data, TIMEOUT))
        expect = np.concatenate([data[1000:101000], data[500000:650000], data[7:50007]])
        np.testing.assert_array_equal(back, expect)
        overlap = (native.Range * 2)(native.Range(0, 0, 100, 0), native.Range(0, 50, 100, 0))
        assert L.gd_read_ranges(ctx, fh, buf, overlap, 2, C.byref(ticket)) == native.E_INVALIDARG
        native.check(L.gd_release_buffer(ctx, buf, TIMEOUT))
        native.check(L.gd_release_file(ctx, fh, TIMEOUT))
    finally:
        os.unlink(path)


def test_unassigned_table_index_is_a_host_error():
    """Every table entry that names no buffer (index 0 among them) points at a zeroed 1 MiB guard
    block, never at address 0 (gd_create reads the table back to make sure), so a dispatch given a
    wrong table index writes into that block instead of faulting the GPU. A context created with
    enable_debug reports such a write from gd_wait_compute as E_FAIL and clears the block: the
    next wait on clean work succeeds. Here a bit-exact copy of 1024 words (4 KiB, inside the
    block) targets index 0 as if the caller had dropped a constant."""
    L = native.lib()
    opts = native.Options(0, 1, 0, 32 << 20, 1024)  # enable_debug
    h = C.c_void_p()
    native.check(L.gd_create(C.byref(opts), C.byref(h)), "gd_create")
    try:
        pipe = C.c_void_p()
        ew = code("ew")
        native.check(L.gd_create_pipeline(h, ew, len(ew), C.byref(pipe)))
        src, sinfo = make_resource(h, 4096, 1)
        dst, dinfo = make_resource(h, 4096, 0)
        data = (np.arange(1024, dtype=np.uint32) | 1).astype(np.uint32)  # every word nonzero
        C.memmove(sinfo.mapped, data.ctypes.data, 4096)
        ticket = C.c_uint64()

        def copy_to(index):
            native.check(L.gd_begin(h, TIMEOUT))
            cst = (C.c_uint32 * 12)(sinfo.uav_index, 0, 0, sinfo.uav_index, 0, 0, index, 0, 0, 1024, 1, 5)
            native.check(L.gd_dispatch(h, pipe, cst, 12, 4, 1, 1))
            native.check(L.gd_submit(h, C.byref(ticket)))
            return L.gd_wait_compute(h, ticket, TIMEOUT)

        assert copy_to(dinfo.uav_index) == 0
        assert copy_to(0) == native.E_FAIL  # the write landed in the guard block
        assert copy_to(dinfo.uav_index) == 0  # the block was cleared
        back = np.zeros(1024, np.uint32)
        native.check(L.gd_readback(h, dst, 0, 4096, back.ctypes.data, TIMEOUT))
        np.testing.assert_array_equal(back, data)
        native.check(L.gd_release_buffer(h, dst, TIMEOUT))
        native.check(L.gd_release_buffer(h, src, TIMEOUT))
        native.check(L.gd_release_pipeline(h, pipe, TIMEOUT))
    finally:
        native.check(L.gd_destroy(h, TIMEOUT), "gd_destroy")
