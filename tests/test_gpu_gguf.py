"""A MoE layer loaded from a GGUF file (include/gyro_gguf.h; src/gguf.zig:138-143 expert slices,
:182-250 rotation metadata, src/model.zig:262-333 counts and signs) runs the decode and prefill
paths: a synthetic layer at the real model's expert shapes (hidden 2560, F 640, top-10, explicit
Hadamard signs) is written with its fp32 router, experts and metadata, read back by
gyrodx.gguf.load_layer, and its outputs must equal, bit for bit, those of the same layer uploaded
from memory, and match the CPU oracle (relative RMS 2e-3, cosine 0.9999)."""
import numpy as np
import pytest

from gguf_fixture import write_layer_file
from gyrodx import gguf, synth
from gyrodx.engine import PATH_DECODE, PATH_PREFILL, Engine

pytestmark = pytest.mark.gpu


def test_layer_from_gguf_decode_and_prefill(tmp_path, oracle_mod):
    L = synth.make_layer(901, E=2560, F=640, n_expert=64, n_used=10)
    L.expert_weights_scale = 2.5
    path = tmp_path / "layer.gguf"
    write_layer_file(path, L)
    G = gguf.load_layer(str(path), 0)
    assert (G.E, G.F, G.n_expert, G.n_used, G.expert_weights_scale) == (L.E, L.F, L.n_expert, L.n_used, 2.5)
    np.testing.assert_array_equal(G.router, L.router)
    np.testing.assert_array_equal(G.gate_signs, L.gate_signs)
    np.testing.assert_array_equal(G.down_signs, L.down_signs)
    x = synth.make_tokens(902, 24, L.E, bf16=True)
    ref, _ = oracle_mod.OracleLayer(L).forward(x, trace=True)
    for path_id, n, name in ((PATH_DECODE, 4, "decode"), (PATH_PREFILL, 24, "prefill")):
        outs = []
        for layer in (L, G):
            eng = Engine(max_tok=24)
            try:
                eng.add_layer(layer)
                outs.append(eng.forward(0, x[:n], path_id))
            finally:
                eng.close()
        np.testing.assert_array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
        r, c = oracle_mod.rel_rms(ref[:n], outs[1]), oracle_mod.cosine(ref[:n], outs[1])
        print(f"gguf layer {name}: rel_rms={r:.3e} cosine={c:.8f}", flush=True)
        assert r <= 2e-3 and c >= 0.9999, (name, r, c)


def test_complete_coder_layer_with_q8_shared_expert(tmp_path, oracle_mod):
    """A complete layer at the real model's shapes as the reference binds it (src/gpu_engine.zig:
    397-401): router, TQ2_T experts at hidden 2560 / F 640 / top-10, and a Q8_0 shared expert of
    width 640 with its fp32 gate, read from one GGUF file; decode and prefill outputs equal those
    of the in-memory layer bit for bit and match the oracle."""
    L = synth.make_layer(911, E=2560, F=640, n_expert=64, n_used=10, SF=640, sh_type=8)
    path = tmp_path / "coder_layer.gguf"
    write_layer_file(path, L)
    G = gguf.load_layer(str(path), 0)
    assert (G.SF, G.sh_type) == (640, 8)
    x = synth.make_tokens(912, 32, L.E, bf16=True)
    ref, _ = oracle_mod.OracleLayer(L).forward(x, trace=True)
    for path_id, n, name in ((PATH_DECODE, 3, "decode"), (PATH_PREFILL, 32, "prefill")):
        outs = []
        for layer in (L, G):
            eng = Engine(max_tok=32)
            try:
                eng.add_layer(layer)
                outs.append(eng.forward(0, x[:n], path_id))
            finally:
                eng.close()
        np.testing.assert_array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
        r, c = oracle_mod.rel_rms(ref[:n], outs[1]), oracle_mod.cosine(ref[:n], outs[1])
        print(f"gguf coder layer + q8 shared {name}: rel_rms={r:.3e} cosine={c:.8f}", flush=True)
        assert r <= 2e-3 and c >= 0.9999, (name, r, c)
