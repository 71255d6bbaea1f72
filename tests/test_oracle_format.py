"""Pins the oracle's Gyro decoder and rotation (CPU only).

Checks mirror the reference's own tests: the codebook hash and fail-closed lengths
(src/gyro.zig:197-214), binary16 edge bits (:216-224), rotation order (:226-238), the 512-block
golden fixture from the independent C oracle (tests/gyro_vectors.zig:28-60), and the
specification's worked examples (third_party/agention-gyro/SPEC.md:337-436). Closed forms of
the Hadamard transform and the reference's own vendored C decoder (built into oracle/_ref when
the reference tree is present) close the rest.
"""
import hashlib
import json
import struct
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"
CODEBOOK = Path(__file__).resolve().parents[1] / "gyro-dx_amd" / "data" / "gyro_codebook.f16"
TYPES = [(144, 34), (145, 26), (146, 30), (147, 42), (148, 50), (149, 58), (150, 22), (151, 18)]


def test_codebook_hash():
    # src/gyro.zig:197-202 and SPEC.md section 4.
    assert hashlib.sha256(CODEBOOK.read_bytes()).hexdigest() == \
        "ee481f151d8947ce8b08817fdf89d0a56d647b6435ceb3df0f079ea748e0e588"


def test_fixture_hash():
    meta = json.loads((GOLDEN / "gyro_vectors.json").read_text())
    assert hashlib.sha256((GOLDEN / "gyro_vectors.bin").read_bytes()).hexdigest() == meta["sha256"]


def parse_fixture():
    """tests/gyro_vectors.zig:28-60 layout."""
    blob = (GOLDEN / "gyro_vectors.bin").read_bytes()
    pos = 0

    def take(n):
        nonlocal pos
        out = blob[pos:pos + n]
        assert len(out) == n
        pos += n
        return out

    def word():
        return struct.unpack("<I", take(4))[0]

    assert take(8) == b"GYROV1\x00\x00"
    cases = []
    for _ in range(word()):
        type_id, size = word(), word()
        enc = take(size)
        bits = np.frombuffer(take(512), dtype="<u4").copy()
        cases.append((type_id, enc, bits))
    rots = []
    for _ in range(word()):
        width, block = word(), word()
        vals = np.frombuffer(take(4 * width), dtype="<f4").copy()
        signs = np.frombuffer(take(width), dtype=np.int8).copy()
        rot = np.frombuffer(take(4 * width), dtype="<u4").copy()
        unrot = np.frombuffer(take(4 * width), dtype="<u4").copy()
        rots.append((width, block, vals, signs, rot, unrot))
    assert pos == len(blob)
    return cases, rots


def test_golden_decode_all_bits(oracle_mod):
    cases, _ = parse_fixture()
    assert len(cases) == 512
    for type_id, enc, bits in cases:
        rc, out = oracle_mod.decode_row(type_id, np.frombuffer(enc, np.uint8), 128)
        assert rc == 0
        np.testing.assert_array_equal(out.view(np.uint32), bits)


def test_golden_rotation_bits(oracle_mod):
    _, rots = parse_fixture()
    assert [r[0] for r in rots] == [640, 2560]
    for width, block, vals, signs, rot, unrot in rots:
        rc, r = oracle_mod.rotate(vals, block, signs)
        assert rc == 0
        np.testing.assert_array_equal(r.view(np.uint32), rot)
        rc, u = oracle_mod.rotate(r, block, signs, inverse=True)
        assert rc == 0
        np.testing.assert_array_equal(u.view(np.uint32), unrot)


def test_fp16_edges(oracle_mod):
    # src/gyro.zig:216-224.
    f = oracle_mod.lib().go_fp16_to_fp32
    as_bits = lambda v: struct.unpack("<I", struct.pack("<f", v))[0]
    assert as_bits(f(0)) == 0x00000000
    assert as_bits(f(0x8000)) == 0x80000000
    assert as_bits(f(1)) == 0x33800000
    assert as_bits(f(0x0400)) == 0x38800000
    assert f(0x7BFF) == 65504.0
    assert np.isinf(f(0x7C00))
    assert np.isnan(f(0x7E00))
    # Every binary16 pattern against numpy's exact conversion.
    allh = np.arange(65536, dtype=np.uint16)
    ref = allh.view(np.float16).astype(np.float32)
    mine = np.array([f(int(h)) for h in range(0, 65536, 97)], dtype=np.float32)
    sel = ref[::97]
    fin = np.isfinite(sel)
    np.testing.assert_array_equal(mine[fin].view(np.uint32), sel[fin].view(np.uint32))


def test_fail_closed(oracle_mod):
    # src/gyro.zig:204-214.
    L = oracle_mod.lib()
    assert L.go_row_bytes(35, 128) == 0
    assert L.go_row_bytes(144, 127) == 0
    assert L.go_row_bytes(144, 640 * 2560) == 435200
    src = np.zeros(34, np.uint8)
    assert oracle_mod.decode_row(144, src, 128, state_bits=-1)[0] == -2
    assert oracle_mod.decode_row(144, src, 128, state_bits=16)[0] == -3
    assert oracle_mod.decode_row(144, src[:33], 128)[0] == -5
    assert oracle_mod.decode_row(35, src, 128)[0] == -1


def test_rotation_order_and_invalid():
    # src/gyro.zig:226-238 and SPEC.md section 10.4.
    import oracle
    signs = np.array([1, -1, 1, 1], np.int8)
    rc, v = oracle.rotate(np.array([1, 2, 3, 4], np.float32), 4, signs)
    assert rc == 0 and v.tolist() == [3, 1, -4, 2]
    rc, v = oracle.rotate(v, 4, signs, inverse=True)
    assert rc == 0 and v.tolist() == [1, 2, 3, 4]
    assert oracle.rotate(v, 3, None)[0] == -7
    assert oracle.rotate(np.ones(4, np.float32), 4, np.array([1, -1, 0, 1], np.int8))[0] == -9


def test_spec_worked_examples(oracle_mod):
    """SPEC.md section 10: states, codebook indices and decoded values of three blocks."""
    kat = json.loads((GOLDEN / "spec_kat.json").read_text())
    L = oracle_mod.lib()
    import ctypes as C
    for case in kat["cases"]:
        enc = np.array(case["bytes"], np.uint8)
        type_id = case["type_id"]
        assert L.go_fp16_to_fp32(int(enc[0]) | int(enc[1]) << 8) == case["d"]
        rc, out = oracle_mod.decode_row(type_id, enc, 128)
        assert rc == 0
        stream = np.ascontiguousarray(enc[2:])
        per = 2 if type_id in (147, 148, 149) else 4
        assert len(case["rows"]) >= 5
        for row in case["rows"]:
            t = row["t"]
            s = L.go_trellis_state(type_id, stream.ctypes.data_as(C.POINTER(C.c_uint8)), t)
            assert s == row["state"]
            h = ((s & 0x7FFF) * 0x9E3779B1) & 0xFFFFFFFF
            assert h >> 21 == row["idx0"]
            if "idx1" in row:
                assert (h >> 10) & 2047 == row["idx1"]
            np.testing.assert_allclose(out[t * per:(t + 1) * per], row["w"], atol=5e-7)


def test_against_vendored_reference_decoder(oracle_mod):
    """Bit-exact agreement with third_party/agention-gyro tq_dequantize_row on random blocks."""
    ref = oracle_mod.ref_lib()
    if ref is None:
        pytest.skip("oracle/_ref not built (reference tree absent)")
    import ctypes as C
    g = np.random.default_rng(7)
    for type_id, bb in TYPES:
        blocks = 300
        raw = g.integers(0, 256, size=(blocks, bb), dtype=np.uint8)
        half = g.integers(0, 65536, size=blocks).astype(np.uint16)
        half[(half & 0x7C00) == 0x7C00] &= 0xBBFF  # finite scales
        raw[:, 0], raw[:, 1] = half & 0xFF, half >> 8
        raw = np.ascontiguousarray(raw.reshape(-1))
        rc, mine = oracle_mod.decode_row(type_id, raw, blocks * 128)
        assert rc == 0
        theirs = np.empty(blocks * 128, np.float32)
        assert ref.tq_dequantize_row(type_id, raw.ctypes.data, theirs.ctypes.data_as(C.POINTER(C.c_float)), blocks * 128) == 0
        np.testing.assert_array_equal(mine.view(np.uint32), theirs.view(np.uint32))
    # Rotation of random widths against the vendored transform.
    for width in (128, 512, 2048):
        v = g.standard_normal(width).astype(np.float32)
        s = (g.integers(0, 2, width) * 2 - 1).astype(np.int8)
        rc, mine = oracle_mod.rotate(v, 128, s)
        theirs = v.copy()
        ref.tq_hadamard_rotate(theirs.ctypes.data_as(C.POINTER(C.c_float)), width, 128, s.ctypes.data_as(C.POINTER(C.c_int8)))
        np.testing.assert_array_equal(mine.view(np.uint32), theirs.view(np.uint32))


def hadamard_matrix(b):
    r = np.arange(b)
    pc = np.vectorize(lambda v: bin(v).count("1"))(r[:, None] & r[None, :])
    return ((-1.0) ** pc) / np.sqrt(b)


def test_rotation_closed_forms(oracle_mod):
    """T v = H_b (s . v) with H_b[r][c] = (-1)^popcount(r&c)/sqrt(b); H H = I; (Tw).(Tx) = w.x."""
    g = np.random.default_rng(3)
    H = hadamard_matrix(128)
    np.testing.assert_allclose(H @ H, np.eye(128), atol=1e-12)
    v = g.standard_normal(384).astype(np.float32)
    w = g.standard_normal(384).astype(np.float32)
    s = (g.integers(0, 2, 384) * 2 - 1).astype(np.int8)
    _, rv = oracle_mod.rotate(v, 128, s)
    _, rw = oracle_mod.rotate(w, 128, s)
    expect = (H @ (s.astype(np.float64) * v).reshape(3, 128).T).T.reshape(-1)
    np.testing.assert_allclose(rv, expect, rtol=0, atol=2e-6)
    assert abs(float(np.dot(rv.astype(np.float64), rw)) - float(np.dot(v.astype(np.float64), w))) < 1e-4


def test_fused_dot_matches_strict_decoder(oracle_mod):
    """src/kernels.zig:384-403: for every type, the fused dot equals decode-then-dot to 1e-4."""
    import ctypes as C
    L = oracle_mod.lib()
    g = np.random.default_rng(7)
    for type_id, bb in TYPES:
        raw = g.integers(0, 256, size=(2, bb), dtype=np.uint8)
        raw[:, 0], raw[:, 1] = 0x00, 0x28  # binary16 0.03125
        raw = np.ascontiguousarray(raw.reshape(-1))
        rc, strict = oracle_mod.decode_row(type_id, raw, 256)
        fast = np.empty(256, np.float32)
        L.go_decode_row_fast(type_id, raw.ctypes.data_as(C.POINTER(C.c_uint8)), fast.ctypes.data_as(C.POINTER(C.c_float)), 256)
        np.testing.assert_array_equal(strict.view(np.uint32), fast.view(np.uint32))
        x = (g.random(256) - 0.5).astype(np.float32)
        d = L.go_dot_row(type_id, raw.ctypes.data_as(C.POINTER(C.c_uint8)), x.ctypes.data_as(C.POINTER(C.c_float)), 256)
        assert abs(d - float(np.dot(strict.astype(np.float64), x))) < 1e-4
