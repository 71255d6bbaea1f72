"""The Q8_0 restatement of the oracle (oracle.q8_0_decode_rows, q8_repack), on the CPU: the
reference's known answer (src/kernels.zig:367-381: scales 0.5 and -0.25, quants j - 16 + b, so
w[0] = 0.5 * -16 and the dot agrees with the dense decode), every int8 value and a negative,
subnormal and zero scale decoded to the value binary16 fixes, and the repacked layout decoding
to the same weights."""
import numpy as np

import oracle


def reference_row():
    row = np.zeros(68, np.uint8)
    for b, s in enumerate((0.5, -0.25)):
        row[b * 34:b * 34 + 2] = np.array([s], np.float16).view(np.uint8)
        row[b * 34 + 2:b * 34 + 34] = (np.arange(32) - 16 + b).astype(np.int8).view(np.uint8)
    return row


def test_reference_known_answer():
    w = oracle.q8_0_decode_rows(reference_row(), 1, 64)[0]
    assert w[0] == 0.5 * -16.0 and w[63] == -0.25 * 16.0 and w[32] == -0.25 * -15.0
    x = (np.arange(64) % 7 - 3.0).astype(np.float32)
    expected = sum(0.5 * (j - 16) * x[j] for j in range(32)) + sum(-0.25 * (j - 15) * x[32 + j] for j in range(32))
    assert abs(float(w.astype(np.float64) @ x) - expected) < 1e-4
    # The C oracle's dotRow of type Q8_0 (dotQ8, src/kernels.zig:107-120) gives the same answer.
    import ctypes as C
    row = reference_row()
    got = oracle.lib().go_dot_row(8, row.ctypes.data_as(C.POINTER(C.c_uint8)),
                                  x.ctypes.data_as(C.POINTER(C.c_float)), 64)
    assert abs(got - expected) < 1e-4
    # A planted mistake (the second block's scale taken as +0.25) misses it.
    bad = row.copy()
    bad[34:36] = np.array([0.25], np.float16).view(np.uint8)
    got_bad = oracle.lib().go_dot_row(8, bad.ctypes.data_as(C.POINTER(C.c_uint8)),
                                      x.ctypes.data_as(C.POINTER(C.c_float)), 64)
    assert abs(got_bad - expected) > 1.0


def test_every_quant_and_special_scales():
    scales = np.array([1.0, -2.0, 2 ** -24, 0.0], np.float16)  # 2^-24: the smallest subnormal
    q = np.arange(-128, 128).reshape(8, 32).astype(np.int8)
    blocks = np.zeros((4, 8, 34), np.uint8)
    for i, s in enumerate(scales):
        blocks[i, :, :2] = np.array([s], np.float16).view(np.uint8)
        blocks[i, :, 2:] = q.view(np.uint8)
    w = oracle.q8_0_decode_rows(blocks, 4, 256)
    for i, s in enumerate(scales):
        np.testing.assert_array_equal(w[i], float(s) * np.arange(-128, 128, dtype=np.float32))


def test_repacked_layout_decodes_to_the_same_weights():
    rng = np.random.default_rng(3)
    rows, cols = 5, 192
    src = rng.integers(0, 256, rows * cols // 32 * 34, dtype=np.uint8)
    src.reshape(-1, 34)[:, 1] &= 0x3b  # finite scales
    packed = oracle.q8_repack(src, rows, cols)
    assert packed.shape == (rows, cols + cols // 16)
    np.testing.assert_array_equal(oracle.q8_repacked_decode(packed, rows, cols),
                                  oracle.q8_0_decode_rows(src, rows, cols))
    # Block 1 of row 2: its quants at bytes 32..63 of the row, its scale at cols + 2.
    blk = src.reshape(rows, cols // 32, 34)[2, 1]
    np.testing.assert_array_equal(packed[2, 32:64], blk[2:])
    np.testing.assert_array_equal(packed[2, cols + 2:cols + 4], blk[:2])
