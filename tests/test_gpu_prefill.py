"""GPU parity of the grouped-GEMM prefill path against the CPU oracle, through the C ABI.

Bar: top-k expert ids identical (tokens whose U-th/(U+1)-th fp64 router probabilities lie
within 1e-5 relative are reported and excluded); the counting sort (route_order, order_start)
identical to the oracle's whenever every token is separable; layer outputs within relative
RMS 2e-3 and cosine 0.9999 of the oracle's fp32 results. Shapes cover the full layer with the
Zipf-skewed router, a single token, ragged tile rows, an expert whose segment spans several
128-row tiles, a layer without rotations, the real model's expert shapes (hidden 2560, F 640,
top-10) and other odd down-row block counts and top-k widths.
"""
import numpy as np
import pytest

from gyrodx import synth
from gyrodx.engine import PATH_PREFILL, Engine

pytestmark = pytest.mark.gpu
REL_RMS = 2e-3
COSINE = 0.9999


def separable(oracle_layer, x, U, margin=1e-5):
    logits = oracle_layer.router_f64(x)
    if oracle_layer.layer.router_bias is not None:
        logits = logits + oracle_layer.layer.router_bias.astype(np.float64)
    p = np.exp(logits - logits.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    s = -np.sort(-p, axis=1)
    return (s[:, U - 1] - s[:, U]) > margin * s[:, U - 1]


def check_tiles(tiles, order_start, tm=128):
    """The tile list covers every expert segment exactly once in tiles of <= tm rows: full tiles
    first in expert order, then the partial tiles by decreasing size, ties by expert."""
    start = np.asarray(order_start, np.int64)
    expect_full, expect_part = [], []
    for e in range(len(start) - 1):
        c = int(start[e + 1] - start[e])
        for j in range(c // tm):
            expect_full.append((e, int(start[e]) + j * tm, tm))
        if c % tm:
            expect_part.append((e, int(start[e]) + (c // tm) * tm, c % tm))
    expect_part.sort(key=lambda t: (-t[2], t[0]))
    got = [tuple(int(v) for v in t[:3]) for t in tiles]
    assert got == expect_full + expect_part


def run_case(oracle_mod, layer, x, max_tok, what):
    eng = Engine(max_tok=max_tok)
    try:
        eng.add_layer(layer)
        n = x.shape[0]
        ol = oracle_mod.OracleLayer(layer)
        ref, tr = ol.forward(x, trace=True)
        print(f"{what}: n={n} E={layer.E} F={layer.F} experts={layer.n_expert}", flush=True)
        out = eng.forward(0, x, PATH_PREFILL)
        ids, w = eng.last_routes(n)
        sep = separable(ol, x, layer.n_used)
        print(f"{what}: {int((~sep).sum())} near-tie tokens excluded", flush=True)
        np.testing.assert_array_equal(ids[sep], tr["route_ids"][sep])
        np.testing.assert_allclose(w[sep], tr["route_w"][sep], rtol=2e-5, atol=1e-7)
        order, start = eng.last_sort(n)
        if sep.all():
            np.testing.assert_array_equal(start, tr["order_start"])
            np.testing.assert_array_equal(order, tr["route_order"])
        # Whatever the ties, the sort is the stable counting sort of the routes the GPU chose
        # (src/engine.zig:553-564).
        flat = ids.reshape(-1).astype(np.int64)
        np.testing.assert_array_equal(start, np.concatenate([[0], np.cumsum(np.bincount(flat, minlength=layer.n_expert))]))
        np.testing.assert_array_equal(order, np.argsort(flat, kind="stable"))
        check_tiles(eng.last_tiles(), tr["order_start"] if sep.all() else eng.last_sort(n)[1])
        r, c = oracle_mod.rel_rms(ref, out), oracle_mod.cosine(ref, out)
        print(f"{what}: rel_rms={r:.3e} cosine={c:.8f}", flush=True)
        assert r <= REL_RMS and c >= COSINE, (what, r, c)
        return eng.last_sort(n)
    finally:
        eng.close()


def test_prefill_full_layer_zipf(oracle_mod):
    """The prefill workload's layer (hidden 2048, 256 experts, top-8, F 512, Zipf(1.1) bias)."""
    layer = synth.make_layer(20261201, zipf=1.1)
    x = synth.make_tokens(20261202, 256, bf16=True)
    order, start = run_case(oracle_mod, layer, x, 256, "full zipf")
    counts = np.diff(start.astype(np.int64))
    assert counts.max() > 128  # at least one expert spans several tiles


@pytest.mark.timeout(600)
def test_prefill_config3_1024_tokens(oracle_mod):
    """The prefill configuration itself: 1024 bf16 tokens through the Zipf(1.1)-biased layer."""
    layer = synth.make_layer(20261201, zipf=1.1)
    x = synth.make_tokens(20261203, 1024, bf16=True)
    order, start = run_case(oracle_mod, layer, x, 1024, "config 3, 1024 tokens")
    assert len(order) == 8192


@pytest.mark.timeout(900)
def test_prefill_4096_tokens(oracle_mod):
    """The stack configuration's 4096-token prefill on one layer: 32,768 slots, the largest call
    the sort and tile list accept (n x n_used <= 32768)."""
    layer = synth.make_layer(4910, zipf=1.1)
    x = synth.make_tokens(4911, 4096, bf16=True)
    eng_tiles = run_case(oracle_mod, layer, x, 4096, "4096 tokens")
    assert len(eng_tiles[0]) == 32768


def test_prefill_wide_router_build(oracle_mod, monkeypatch):
    """The wide router build (moe_prefill_router_w, which the engine takes for 2048 tokens and
    more) forced on every call: ragged token counts, 32, 64, 128 and 256 experts (waves and
    column tiles past n_expert idle), hidden 2560 with top-10, a layer without rotations and the
    Zipf layer with its bias, each against the oracle."""
    monkeypatch.setenv("GYRO_ROUTER_WIDE_MIN", "1")
    cases = [
        (synth.make_layer(31, E=1024, F=256, n_expert=64, n_used=8), 37, 64, "64 experts, n=37"),
        (synth.make_layer(41, E=1024, F=256, n_expert=32, n_used=8), 5, 64, "32 experts, n=5"),
        (synth.make_layer(71, E=2560, F=640, n_expert=128, n_used=10, zipf=1.1), 150, 160, "hidden 2560, top-10"),
        (synth.make_layer(51, E=1024, F=512, n_expert=64, n_used=8, signs=False), 70, 128, "no signs"),
        (synth.make_layer(20261201, zipf=1.1), 256, 256, "full zipf"),
    ]
    for layer, n, max_tok, what in cases:
        run_case(oracle_mod, layer, synth.make_tokens(700 + n, n, layer.E, bf16=True), max_tok, f"wide router: {what}")


def test_prefill_single_and_ragged(oracle_mod):
    layer = synth.make_layer(31, E=1024, F=256, n_expert=64, n_used=8)
    for n in (1, 37):
        run_case(oracle_mod, layer, synth.make_tokens(32 + n, n, layer.E, bf16=True), 64, f"ragged n={n}")


def test_prefill_hot_experts_span_tiles(oracle_mod):
    """A steep bias sends every token to the same few experts: segments of 300 rows."""
    layer = synth.make_layer(41, E=1024, F=256, n_expert=32, n_used=8, zipf=1.1, zipf_factor=6.0)
    x = synth.make_tokens(42, 300, layer.E, bf16=True)
    order, start = run_case(oracle_mod, layer, x, 300, "hot experts")
    assert np.diff(start.astype(np.int64)).max() == 300


def test_prefill_coder_shapes_top10(oracle_mod):
    """The real model's expert shapes: hidden 2560, F 640 (five blocks per down row, so odd down
    rows start 2 bytes off a 4-byte boundary), top-10 routing, with a Zipf-skewed router."""
    layer = synth.make_layer(71, E=2560, F=640, n_expert=128, n_used=10, zipf=1.1)
    run_case(oracle_mod, layer, synth.make_tokens(72, 150, layer.E, bf16=True), 160, "coder shapes")


def test_prefill_odd_down_blocks_other_top_k(oracle_mod):
    """F 384 (three blocks per down row) with top-6 and top-16 routing."""
    for U, n in ((6, 53), (16, 21)):
        layer = synth.make_layer(80 + U, E=1024, F=384, n_expert=64, n_used=U)
        run_case(oracle_mod, layer, synth.make_tokens(90 + U, n, layer.E, bf16=True), 64, f"F 384 top-{U}")


def test_prefill_without_rotations(oracle_mod):
    layer = synth.make_layer(51, E=1024, F=512, n_expert=64, n_used=8, signs=False)
    run_case(oracle_mod, layer, synth.make_tokens(52, 70, layer.E), 128, "no signs")


def test_prefill_falls_back_on_fp16_overflowing_scales(oracle_mod):
    """A block whose scale x codebook products overflow binary16 (scale 60000 in one gate block of
    expert 3) keeps the layer off the fp16 grouped GEMMs: gm_forward on the prefill path runs the
    generic path's fp32 kernels instead of refusing, and so does a prefill stack holding the
    layer. Outputs against the oracle, with the outlier expert among the routes."""
    layer = synth.make_layer(61, E=1024, F=256, n_expert=16, n_used=8)
    layer.gate[3][5, 0:2] = np.frombuffer(np.float16(60000.0).tobytes(), np.uint8)
    x = synth.make_tokens(62, 16, layer.E)
    ref = oracle_mod.OracleLayer(layer).forward(x)
    eng = Engine(max_tok=16)
    try:
        eng.add_layer(layer)
        out = eng.forward(0, x, PATH_PREFILL)
        ids, _ = eng.last_routes(16)
        assert (ids == 3).any(), "no token routed to the outlier expert"
        r, c = oracle_mod.rel_rms(ref, out), oracle_mod.cosine(ref, out)
        print(f"prefill with an overflowing block scale: rel_rms {r:.3e} cosine {c:.8f}", flush=True)
        assert r <= REL_RMS and c >= COSINE
        # A two-layer stack: the outlier layer second, a plain layer first.
        S = synth.make_stack(63, 2, E=1024, F=256, n_expert=16, n_used=8)
        S[1].gate[3][5, 0:2] = np.frombuffer(np.float16(60000.0).tobytes(), np.uint8)
        sids = [eng.add_layer(L) for L in S]
        h = x.copy()
        for L in S:
            h = h + oracle_mod.OracleLayer(L).forward(oracle_mod.rms_norm(h, L.norm_weight, L.norm_eps))
        got = eng.forward_stack(sids, x, PATH_PREFILL)
        r = oracle_mod.rel_rms(h, got)
        print(f"prefill stack with the outlier layer: rel_rms {r:.3e}", flush=True)
        assert r <= REL_RMS
    finally:
        eng.close()
