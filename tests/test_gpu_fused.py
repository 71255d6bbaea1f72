"""moe_decode_fused, the single-launch batch-1 decode path of uniform TQ2_T layers, through the C
ABI, against the CPU oracle (src/engine.zig:520-653 for the layer, src/kernels.zig:281-291 for a
stack's RMSNorm).

Engines created with GYRO_DECODE_FUSED=2 fail any batch-1 decode call that the fused kernel cannot
take, so these outputs come from it; engines with GYRO_DECODE_FUSED=0 run the three-kernel path on
the same tokens. Bar: top-k ids equal to the oracle's for every token whose U-th and (U+1)-th
router probabilities are separated by more than 1e-5 relative, weights within 2e-5 relative, and
outputs within relative RMS 2e-3 and cosine 0.9999 of the oracle's fp32 results. Shapes cover the
configuration-2 layer, the real model's expert shape (hidden 2560, F 640, top-10), the largest
hidden width (4096) and F (1024), top-1 and top-16, four gate/up units per group, fewer router
rows than workgroups (the arrival words), no sign vectors and a router-logit bias.
"""
import os

import numpy as np
import pytest

from gyrodx import synth
from gyrodx.engine import PATH_DECODE, Engine

pytestmark = pytest.mark.gpu
REL_RMS = 2e-3
COSINE = 0.9999


def make_engine(max_tok, mode, spin_limit=None):
    """An engine whose batch-1 decode mode is `mode` (GYRO_DECODE_FUSED, read at gm_create)."""
    saved = {k: os.environ.get(k) for k in ("GYRO_DECODE_FUSED", "GYRO_DECODE_SPIN_LIMIT")}
    os.environ["GYRO_DECODE_FUSED"] = mode
    if spin_limit is not None:
        os.environ["GYRO_DECODE_SPIN_LIMIT"] = str(spin_limit)
    try:
        return Engine(max_tok=max_tok)
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


def separable(ol, x, U, margin=1e-5):
    logits = ol.router_f64(x)
    p = np.exp(logits - logits.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    s = -np.sort(-p, axis=1)
    return (s[:, U - 1] - s[:, U]) > margin * s[:, U - 1]


def close(oracle_mod, ref, out, what):
    assert np.isfinite(out).all(), what
    r, c = oracle_mod.rel_rms(ref, out), oracle_mod.cosine(ref, out)
    print(f"{what}: rel_rms={r:.3e} cosine={c:.8f}", flush=True)
    assert r <= REL_RMS and c >= COSINE, (what, r, c)
    return r


SHAPES = [
    # E, F, experts, top-k, extra make_layer arguments
    (2048, 512, 256, 8, {}),
    (2560, 640, 128, 10, {}),
    (4096, 256, 32, 4, {}),
    (256, 1024, 32, 16, {}),
    (1024, 384, 64, 6, {}),
    (2048, 512, 64, 1, {}),
    (512, 256, 8, 2, {}),
    (1024, 512, 64, 8, {"signs": False}),
    (1024, 512, 64, 8, {"zipf": 1.1}),
]


@pytest.mark.parametrize("E,F,NE,U,kw", SHAPES, ids=[f"E{s[0]}-F{s[1]}-x{s[2]}-top{s[3]}-{'-'.join(s[4]) or 'signs'}"
                                                    for s in SHAPES])
def test_fused_decode_parity(oracle_mod, E, F, NE, U, kw):
    L = synth.make_layer(900 + E // 128 + F // 64 + U, E=E, F=F, n_expert=NE, n_used=U, **kw)
    ol = oracle_mod.OracleLayer(L)
    n = 6
    x = synth.make_tokens(901 + U, n, E)
    ref, tr = ol.forward(x, trace=True)
    sep = separable(ol, x, U)
    fused, three = make_engine(4, "2"), make_engine(4, "0")
    try:
        fused.add_layer(L)
        three.add_layer(L)
        print(f"fused decode E={E} F={F} experts={NE} top-{U} {kw}: {n} tokens, "
              f"{int((~sep).sum())} near a routing tie", flush=True)
        worst = 0.0
        for t in range(n):
            out = fused.forward(0, x[t:t + 1], PATH_DECODE)
            ids, w = fused.last_routes(1)
            if sep[t]:
                np.testing.assert_array_equal(ids[0], tr["route_ids"][t])
                np.testing.assert_allclose(w[0], tr["route_w"][t], rtol=2e-5, atol=1e-7)
            worst = max(worst, close(oracle_mod, ref[t], out[0], f"  fused token {t}"))
            o3 = three.forward(0, x[t:t + 1], PATH_DECODE)
            close(oracle_mod, ref[t], o3[0], f"  three-kernel token {t}")
        print(f"fused decode E={E} F={F} top-{U}: worst rel_rms {worst:.3e}", flush=True)
    finally:
        fused.close()
        three.close()


def test_fused_run_matches_forward(oracle_mod):
    """gm_run over 40 device-resident tokens, cycling two layers (40 calls: epochs and counters
    carried from call to call), equals gm_forward bit for bit; another engine's calls in between
    use their own exchange area."""
    layers = [synth.make_layer(950 + i, E=2048, F=512, n_expert=256, n_used=8) for i in range(2)]
    x = synth.make_tokens(952, 40)
    eng, other = make_engine(1, "2"), make_engine(1, "2")
    try:
        ids = [eng.add_layer(L) for L in layers]
        other.add_layer(layers[1])
        eng.set_tokens(x)
        print("fused gm_run: 40 calls over 2 layers", flush=True)
        dev_ms, wall_ms, _ = eng.run(PATH_DECODE, 1, 40, ids)
        got = eng.read_outputs(40)
        assert dev_ms > 0 and wall_ms > 0
        for t in (0, 1, 17, 38, 39):
            one = eng.forward(ids[t % 2], x[t:t + 1], PATH_DECODE)
            np.testing.assert_array_equal(got[t].view(np.uint32), one[0].view(np.uint32), err_msg=f"token {t}")
            two = other.forward(0, x[t:t + 1], PATH_DECODE)
            if t % 2 == 1:
                np.testing.assert_array_equal(two[0].view(np.uint32), one[0].view(np.uint32), err_msg=f"token {t}")
        ref = oracle_mod.OracleLayer(layers[0]).forward(x[:4:2])
        close(oracle_mod, ref, got[:4:2], "fused gm_run tokens 0, 2")
    finally:
        eng.close()
        other.close()


def test_fused_stack_norm(oracle_mod):
    """A three-layer stack at batch 1 (RMSNorm with and without weight inside the fused kernel,
    the residual added by its combine, in place): gm_forward_stack against the oracle's stack,
    and gm_run_stack over 4 tokens equal to it bit for bit."""
    layers = synth.make_stack(960, 3, E=2048, F=512, n_expert=128, n_used=8)
    layers[1].norm_weight = None
    x = synth.make_tokens(961, 4)
    eng = make_engine(1, "2")
    try:
        ids = [eng.add_layer(L) for L in layers]
        print("fused stack: 3 layers, 4 tokens one at a time", flush=True)
        outs = []
        for t in range(4):
            h = x[t:t + 1].copy()
            for L in layers:
                ol = oracle_mod.OracleLayer(L)
                h = h + ol.forward(oracle_mod.rms_norm(h, L.norm_weight, L.norm_eps))
            out = eng.forward_stack(ids, x[t:t + 1], PATH_DECODE)
            outs.append(out)
            close(oracle_mod, h, out, f"  fused stack token {t}")
        eng.set_tokens(x)
        eng.run_stack(PATH_DECODE, 1, 4, ids)
        got = eng.read_outputs(4)
        for t in range(4):
            np.testing.assert_array_equal(got[t].view(np.uint32), outs[t][0].view(np.uint32), err_msg=f"token {t}")
    finally:
        eng.close()


def test_fused_wait_limit_recovers(oracle_mod):
    """A spin limit of 0 makes the kernel's waits give up at their first unready poll (the
    condition forced from the host; every wait stays bounded, so the grid drains): gm_forward
    recomputes the call on the three-kernel path, a timed gm_run raises, and the exchange area
    is clean for the next calls."""
    L = synth.make_layer(970, E=2048, F=512, n_expert=256, n_used=8)
    x = synth.make_tokens(971, 4)
    ref = oracle_mod.OracleLayer(L).forward(x)
    eng = make_engine(1, "1", spin_limit=0)
    try:
        eng.add_layer(L)
        print("fused decode with spin limit 0: gm_forward falls back", flush=True)
        close(oracle_mod, ref[0], eng.forward(0, x[:1], PATH_DECODE)[0], "  spin limit 0, gm_forward")
        eng.set_tokens(x)
        with pytest.raises(RuntimeError, match="gave up"):
            eng.run(PATH_DECODE, 1, 4, [0])
    finally:
        eng.close()
    # A normal engine on the same GPU afterwards.
    eng = make_engine(1, "2")
    try:
        eng.add_layer(L)
        for t in range(2):
            close(oracle_mod, ref[t], eng.forward(0, x[t:t + 1], PATH_DECODE)[0], f"  after the give-ups, token {t}")
    finally:
        eng.close()
