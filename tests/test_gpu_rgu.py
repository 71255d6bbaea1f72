"""moe_decode_rgu, the decode path's router, input rotation, routing and gate/up in one launch,
through the C ABI.

moe_decode_rgu keeps moe_router's arithmetic for the logits, the norm and the rotation and then
runs moe_decode_gu's body, so an engine that takes it (created with GYRO_DECODE_RGU=1; the tuned
TQ2_T shapes: hidden 1024 or 2048, F 512, top-8) must give the same bits as an engine created
with GYRO_DECODE_RGU=0 (moe_router, then moe_decode_gu): outputs, top-8 ids and weights. Against the
CPU oracle (src/engine.zig:520-653; src/kernels.zig:281-291 for a stack's RMSNorm) the bar is
that of the decode path: ids equal for every token whose 8th and 9th router probabilities are
separated by more than 1e-5 relative, weights within 2e-5 relative, outputs within relative RMS
2e-3 and cosine 0.9999. Cases: 256 experts at hidden 2048 (one router row per producing group)
and 1024 (two rows), 64 experts (fewer producers than groups), a router bias, no sign vectors,
batches 1, 3 and 8, a three-layer stack with RMSNorm, a Q8_0 shared expert beside the routed
experts, gm_run over many calls (a new epoch each) and a forced give-up of the logit wait.
"""
import os

import numpy as np
import pytest

from gyrodx import synth
from gyrodx.engine import PATH_DECODE, Engine

pytestmark = pytest.mark.gpu
REL_RMS = 2e-3
COSINE = 0.9999


def make_engine(max_tok, rgu, spin_limit=None):
    """An engine with moe_decode_rgu on (rgu='1') or off ('0'); the spin limit of its waits."""
    saved = {k: os.environ.get(k) for k in ("GYRO_DECODE_RGU", "GYRO_DECODE_SPIN_LIMIT", "GYRO_DECODE_FUSED")}
    os.environ["GYRO_DECODE_RGU"] = rgu
    os.environ["GYRO_DECODE_FUSED"] = "0"
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


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


SHAPES = [
    # E, experts, make_layer arguments
    (2048, 256, {}),
    (1024, 256, {}),
    (2048, 64, {}),
    (2048, 256, {"zipf": 1.1}),
    (1024, 128, {"signs": False}),
]


@pytest.mark.parametrize("E,NE,kw", SHAPES, ids=[f"E{s[0]}-x{s[1]}-{'-'.join(s[2]) or 'signs'}" for s in SHAPES])
def test_rgu_matches_three_kernel_path(oracle_mod, E, NE, kw):
    L = synth.make_layer(1200 + E // 256 + NE // 32, E=E, F=512, n_expert=NE, n_used=8, **kw)
    ol = oracle_mod.OracleLayer(L)
    x = synth.make_tokens(1201 + NE, 12, E)
    ref, tr = ol.forward(x, trace=True)
    sep = separable(ol, x, 8)
    rgu, three = make_engine(8, "1"), make_engine(8, "0")
    try:
        rgu.add_layer(L)
        three.add_layer(L)
        print(f"rgu decode E={E} experts={NE} {kw}: 12 tokens at batches 1, 3, 8; "
              f"{int((~sep).sum())} near a routing tie", flush=True)
        t0 = 0
        for n in (1, 3, 8):
            xs = x[t0:t0 + n]
            out = rgu.forward(0, xs, PATH_DECODE)
            ids, w = rgu.last_routes(n)
            o3 = three.forward(0, xs, PATH_DECODE)
            ids3, w3 = three.last_routes(n)
            np.testing.assert_array_equal(bits(out), bits(o3), err_msg=f"outputs, batch {n}")
            np.testing.assert_array_equal(ids, ids3, err_msg=f"ids, batch {n}")
            np.testing.assert_array_equal(bits(w), bits(w3), err_msg=f"weights, batch {n}")
            for i in range(n):
                t = t0 + i
                if sep[t]:
                    np.testing.assert_array_equal(ids[i], tr["route_ids"][t])
                    np.testing.assert_allclose(w[i], tr["route_w"][t], rtol=2e-5, atol=1e-7)
            close(oracle_mod, ref[t0:t0 + n], out, f"  batch {n}, tokens {t0}..{t0 + n - 1}")
            t0 += n
    finally:
        rgu.close()
        three.close()


def test_rgu_stack_norm(oracle_mod):
    """A three-layer stack (RMSNorm with and without weight, computed inside moe_decode_rgu; the
    residual added by moe_decode_down) at batch 1 and 8: gm_forward_stack bit-equal to the
    three-kernel engine and within the bar of the oracle's stack; gm_run_stack equal to it."""
    layers = synth.make_stack(1260, 3, E=2048, F=512, n_expert=256, n_used=8)
    layers[1].norm_weight = None
    x = synth.make_tokens(1261, 9)
    rgu, three = make_engine(8, "1"), make_engine(8, "0")
    try:
        ids = [rgu.add_layer(L) for L in layers]
        ids3 = [three.add_layer(L) for L in layers]
        print("rgu stack: 3 layers, a batch of 1 and a batch of 8", flush=True)
        h = x.copy()
        for L in layers:
            h = h + oracle_mod.OracleLayer(L).forward(oracle_mod.rms_norm(h, L.norm_weight, L.norm_eps))
        for lo, hi in ((0, 1), (1, 9)):
            out = rgu.forward_stack(ids, x[lo:hi], PATH_DECODE)
            o3 = three.forward_stack(ids3, x[lo:hi], PATH_DECODE)
            np.testing.assert_array_equal(bits(out), bits(o3), err_msg=f"stack batch {hi - lo}")
            close(oracle_mod, h[lo:hi], out, f"  rgu stack batch {hi - lo}")
        rgu.set_tokens(x[1:9])
        rgu.run_stack(PATH_DECODE, 8, 1, ids)
        got = rgu.read_outputs(8)
        np.testing.assert_array_equal(bits(got), bits(rgu.forward_stack(ids, x[1:9], PATH_DECODE)))
    finally:
        rgu.close()
        three.close()


def test_rgu_with_q8_shared_expert(oracle_mod):
    """A Q8_0 shared expert of width 640 runs in the matrix-vector kernels before the routed
    experts and enters moe_decode_down as its residual input; the routed part takes
    moe_decode_rgu. Bit-equal to the three-kernel engine, within the bar of the oracle."""
    L = synth.make_layer(1270, E=2048, F=512, n_expert=256, n_used=8, SF=640, sh_type=8)
    x = synth.make_tokens(1271, 4)
    ref = oracle_mod.OracleLayer(L).forward(x)
    rgu, three = make_engine(4, "1"), make_engine(4, "0")
    try:
        rgu.add_layer(L)
        three.add_layer(L)
        print("rgu decode with a Q8_0 shared expert (SF 640): batch 1 and 3", flush=True)
        for lo, hi in ((0, 1), (1, 4)):
            out = rgu.forward(0, x[lo:hi], PATH_DECODE)
            np.testing.assert_array_equal(bits(out), bits(three.forward(0, x[lo:hi], PATH_DECODE)))
            close(oracle_mod, ref[lo:hi], out, f"  shared Q8_0, batch {hi - lo}")
    finally:
        rgu.close()
        three.close()


def test_rgu_run_matches_forward(oracle_mod):
    """gm_run over 40 device-resident tokens, cycling two layers (a new epoch per call), equals
    gm_forward bit for bit; another engine's calls in between use their own logit words."""
    layers = [synth.make_layer(1280 + i, E=2048, F=512, n_expert=256, n_used=8) for i in range(2)]
    x = synth.make_tokens(1282, 40)
    eng, other = make_engine(1, "1"), make_engine(1, "1")
    try:
        ids = [eng.add_layer(L) for L in layers]
        other.add_layer(layers[1])
        eng.set_tokens(x)
        print("rgu gm_run: 40 calls over 2 layers", flush=True)
        dev_ms, wall_ms, _ = eng.run(PATH_DECODE, 1, 40, ids)
        got = eng.read_outputs(40)
        assert dev_ms > 0 and wall_ms > 0
        for t in (0, 1, 17, 38, 39):
            one = eng.forward(ids[t % 2], x[t:t + 1], PATH_DECODE)
            np.testing.assert_array_equal(bits(got[t]), bits(one[0]), err_msg=f"token {t}")
            two = other.forward(0, x[t:t + 1], PATH_DECODE)
            if t % 2 == 1:
                np.testing.assert_array_equal(bits(two[0]), bits(one[0]), err_msg=f"token {t}")
        ref = oracle_mod.OracleLayer(layers[0]).forward(x[:4:2])
        close(oracle_mod, ref, got[:4:2], "rgu gm_run tokens 0, 2")
    finally:
        eng.close()
        other.close()


def test_rgu_wait_limit_recovers(oracle_mod):
    """A spin limit of 0 makes the logit wait give up at its first unready poll (forced from the
    host; the wait stays bounded, so the grid drains): gm_forward recomputes the call on the
    three-kernel path, a timed gm_run raises, and the next engine's calls are clean."""
    L = synth.make_layer(1290, E=2048, F=512, n_expert=256, n_used=8)
    x = synth.make_tokens(1291, 4)
    ref = oracle_mod.OracleLayer(L).forward(x)
    eng = make_engine(1, "1", spin_limit=0)
    try:
        eng.add_layer(L)
        print("rgu decode with spin limit 0: gm_forward falls back", flush=True)
        close(oracle_mod, ref[0], eng.forward(0, x[:1], PATH_DECODE)[0], "  spin limit 0, gm_forward")
        eng.set_tokens(x)
        with pytest.raises(RuntimeError, match="gave up"):
            eng.run(PATH_DECODE, 1, 4, [0])
    finally:
        eng.close()
    eng = make_engine(1, "1")
    try:
        eng.add_layer(L)
        for t in range(2):
            close(oracle_mod, ref[t], eng.forward(0, x[t:t + 1], PATH_DECODE)[0], f"  after the give-ups, token {t}")
    finally:
        eng.close()
