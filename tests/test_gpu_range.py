"""The activation range guard of the prefill path, through the C ABI: the prefill path rounds
activations to binary16 for its MFMA products (the rotated input in moe_prefill_router, the SwiGLU
output in the prefill gate/up GEMMs and the shared expert); a value outside the binary16 range
sets a flag, gm_forward then recomputes the call on GM_PATH_GENERIC (fp32 activations, the
reference's own arithmetic), and a timed gm_run raises. The decode path keeps every activation in
fp32, so the same inputs run through it directly. Outputs must match the CPU oracle, which keeps
every activation in fp32 (src/engine.zig:520-653)."""
import numpy as np
import pytest

from gyrodx import synth
from gyrodx.engine import PATH_DECODE, PATH_PREFILL, Engine

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def layer():
    return synth.make_layer(701, E=2048, F=512, n_expert=64, n_used=8)


def close(oracle_mod, ref, out, what):
    assert np.isfinite(out).all(), what
    r, c = oracle_mod.rel_rms(ref, out), oracle_mod.cosine(ref, out)
    print(f"{what}: rel_rms={r:.3e} cosine={c:.8f}", flush=True)
    assert r <= 2e-3 and c >= 0.9999, (what, r, c)


def test_outlier_token_recomputed_on_fp32_path(oracle_mod, layer):
    """A token whose rotated input exceeds 65504 (x[0] = 2e6) among ordinary tokens."""
    x = synth.make_tokens(702, 16, layer.E)
    x[3, 0] = 2.0e6
    ref = oracle_mod.OracleLayer(layer).forward(x)
    eng = Engine(max_tok=16)
    try:
        eng.add_layer(layer)
        close(oracle_mod, ref[:4], eng.forward(0, x[:4], PATH_DECODE), "decode with an outlier token")
        close(oracle_mod, ref, eng.forward(0, x, PATH_PREFILL), "prefill with an outlier token")
        # A timed prefill run over the same tokens refuses its outputs; the flag is then clear
        # again. A timed decode run keeps fp32 activations and returns the oracle's outputs.
        eng.set_tokens(x)
        with pytest.raises(RuntimeError, match="binary16 range"):
            eng.run(PATH_PREFILL, 4, 1, [0])
        eng.run(PATH_PREFILL, 3, 1, [0])  # tokens 0..2: in range
        close(oracle_mod, ref[:3], eng.read_outputs(3), "prefill run after the refusal")
        eng.run(PATH_DECODE, 1, 4, [0])
        close(oracle_mod, ref[:4], eng.read_outputs(4), "decode run over the outlier token")
    finally:
        eng.close()


def test_large_activations_in_the_prefill_gemm(oracle_mod, layer):
    """Inputs scaled by 3000: the rotated input fits binary16 but the SwiGLU output of the gate/up
    GEMM does not; the prefill call is recomputed. Decode keeps those activations in fp32."""
    x = synth.make_tokens(703, 12, layer.E) * np.float32(3000.0)
    ref = oracle_mod.OracleLayer(layer).forward(x)
    eng = Engine(max_tok=16)
    try:
        eng.add_layer(layer)
        close(oracle_mod, ref, eng.forward(0, x, PATH_PREFILL), "prefill with large activations")
        close(oracle_mod, ref[:8], eng.forward(0, x[:8], PATH_DECODE), "decode with large activations")
    finally:
        eng.close()
