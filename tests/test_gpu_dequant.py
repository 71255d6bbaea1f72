"""The fast paths' device decoders, bit for bit against the strict decoder (src/gyro.zig:81-105;
src/kernels.zig:384-403 tests the fused decoders against it for all eight types), through
gm_dequant_as, on the GPU:
  - the decode kernels' block decoders (TQ2_T state pairs; gyro_unpack + gyro_kstate),
  - the prefill GEMMs' B-operand decoders for both lane halves (gg_gather; gx_half_stream +
    gx_gather_piece), and
  - the binary16 B operand the MFMA reads, which must equal binary16(strict value) rounded to
    nearest even (the prefill path's one rounding of the weights; its error bound is printed).
Each layer carries the golden fixture's 64 blocks of its type (every scale class: +-0,
subnormals, normals, the largest finite) as the first rows of expert 0's gate (4 blocks per row,
every block start parity) and down (F 640: 5 blocks per row, so odd rows start 2 bytes past a
4-byte boundary) projections, and seeded random blocks elsewhere.
"""
import numpy as np
import pytest

from gyrodx import synth
from gyrodx.engine import Engine
from test_oracle_format import parse_fixture

pytestmark = pytest.mark.gpu
E, F = 512, 640


def strict(oracle_mod, type_id, mat, cols):
    out = np.empty((mat.shape[0], cols), np.float32)
    for r in range(mat.shape[0]):
        rc, out[r] = oracle_mod.decode_row(type_id, mat[r], cols)
        assert rc == 0
    return out


@pytest.mark.parametrize("type_id", sorted(synth.TYPES))
def test_fast_decoders_bit_exact(oracle_mod, type_id):
    layer = synth.make_layer(1000 + type_id, E=E, F=F, n_expert=3, n_used=2, type_id=type_id)
    bb = synth.TYPES[type_id][2]
    blocks = np.frombuffer(b"".join(enc for t, enc, _ in parse_fixture()[0] if t == type_id), np.uint8)
    blocks = blocks.reshape(64, bb)
    gate = layer.gate[0].copy()
    gate[:16] = blocks.reshape(16, 4 * bb)
    down = layer.down[0].copy()
    down[:12] = blocks[:60].reshape(12, 5 * bb)
    layer.gate[0], layer.down[0] = gate, down
    eng = Engine(max_tok=4)
    worst_rel, worst_abs = 0.0, 0.0
    try:
        eng.add_layer(layer)
        for e in range(3):
            for proj, mats in enumerate((layer.gate, layer.up, layer.down)):
                rows, cols = (F, E) if proj < 2 else (E, F)
                ref = strict(oracle_mod, type_id, mats[e], cols)
                for decoder in (0, 1):
                    got = eng.dequant(0, e, proj, 0, rows, cols, decoder)
                    bad = np.flatnonzero(got.view(np.uint32) != ref.view(np.uint32))
                    assert bad.size == 0, (type_id, e, proj, decoder, bad[:4])
                b16 = eng.dequant(0, e, proj, 0, rows, cols, 2)
                expect = ref.astype(np.float16).astype(np.float32)  # round to nearest even
                bad = np.flatnonzero(b16.view(np.uint32) != expect.view(np.uint32))
                assert bad.size == 0, (type_id, e, proj, "binary16", bad[:4])
                fin = np.isfinite(expect) & (np.abs(ref) >= 2.0 ** -14)  # normal binary16 results
                if fin.any():
                    worst_rel = max(worst_rel, float(np.max(np.abs(b16[fin] - ref[fin]) / np.abs(ref[fin]))))
                sub = np.abs(ref) < 2.0 ** -14
                if sub.any():
                    worst_abs = max(worst_abs, float(np.max(np.abs(b16[sub] - ref[sub]))))
    finally:
        eng.close()
    print(f"type {type_id}: decode and prefill decoders bit-exact; binary16 B operand: worst relative error "
          f"{worst_rel:.3e} (normal), worst absolute {worst_abs:.3e} (subnormal)", flush=True)
    assert worst_rel <= 2.0 ** -11 and worst_abs <= 2.0 ** -25
