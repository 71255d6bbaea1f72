"""Routed experts loaded from a GGUF file (include/gyro_gguf.h, src/gguf.zig:138-143) run the
decode and prefill paths: a synthetic layer at the real model's expert shapes (hidden 2560,
F 640, top-10) is written as blk.0.ffn_{gate,up,down}_exps.weight, read back through gg_open and
the expert ranges, and its outputs must equal, bit for bit, those of the same layer uploaded
from memory, and match the CPU oracle (relative RMS 2e-3, cosine 0.9999)."""
import dataclasses

import numpy as np
import pytest

from gguf_fixture import GgufBuilder
from gyrodx import gguf, synth
from gyrodx.engine import PATH_DECODE, PATH_PREFILL, Engine

pytestmark = pytest.mark.gpu


def write_layer(path, L):
    f = GgufBuilder().header(3, 1).kv_u32("general.alignment", 32)
    off, offs, mats = 0, {}, {}
    for p, dims in (("gate", (L.E, L.F, L.n_expert)), ("up", (L.E, L.F, L.n_expert)),
                    ("down", (L.F, L.E, L.n_expert))):
        mats[p] = np.stack(getattr(L, p))
        offs[p] = off
        f.tensor(f"blk.0.ffn_{p}_exps.weight", dims, 144, off)
        off += (mats[p].nbytes + 31) // 32 * 32
    f.pad()
    data = bytearray(off)
    for p in mats:
        data[offs[p]:offs[p] + mats[p].nbytes] = mats[p].tobytes()
    path.write_bytes(f.bytes() + bytes(data))


def test_experts_from_gguf_decode_and_prefill(tmp_path, oracle_mod):
    L = synth.make_layer(901, E=2560, F=640, n_expert=64, n_used=10)
    path = tmp_path / "layer.gguf"
    write_layer(path, L)
    ex = gguf.load_layer_experts(str(path), 0)
    assert (ex["E"], ex["F"], ex["n_expert"]) == (L.E, L.F, L.n_expert)
    G = dataclasses.replace(L, gate=ex["gate"], up=ex["up"], down=ex["down"], types=ex["types"])
    ref, _ = oracle_mod.OracleLayer(L).forward(synth.make_tokens(902, 24, L.E, bf16=True), trace=True)
    x = synth.make_tokens(902, 24, L.E, bf16=True)
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
        print(f"gguf experts {name}: rel_rms={r:.3e} cosine={c:.8f}", flush=True)
        assert r <= 2e-3 and c >= 0.9999, (name, r, c)
