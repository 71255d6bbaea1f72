"""Pins the oracle's MoE layer (src/engine.zig:520-687) on the CPU.

The reference has no test of the layer output (only the decoder and rotation are pinned), so
the layer is pinned by an independent fp64 numpy model written from the algebra: dense
weights from the golden-pinned decoder, the Hadamard matrix in closed form, softmax, brute
force top-k with lower-index ties, and the k-ordered combine. Planted mistakes (a dropped
rotation, a transposed expert index, a wrong tie rule) must fail these checks.
"""
import numpy as np
import pytest

from gyrodx import synth


def dense(oracle_mod, L, e, proj):
    mats = {0: L.gate, 1: L.up, 2: L.down}[proj]
    rows, cols = (L.F, L.E) if proj < 2 else (L.E, L.F)
    t = int(L.types[e, proj])
    rb = synth.row_bytes(t, cols)
    out = np.empty((rows, cols), np.float64)
    for r in range(rows):
        rc, v = oracle_mod.decode_row(t, mats[e][r], cols)
        assert rc == 0
        out[r] = v
    return out


def hadamard_matrix(b):
    r = np.arange(b)
    pc = np.array([[bin(i & j).count("1") for j in r] for i in r])
    return ((-1.0) ** pc) / np.sqrt(b)


def rotate64(v, signs, H):
    v = v * (signs if signs is not None else 1.0)
    b = H.shape[0]
    return (v.reshape(-1, b) @ H.T).reshape(v.shape)


def numpy_layer(oracle_mod, L, x, drop_down_rotation=False, swap_expert=False, tie_high=False):
    H = hadamard_matrix(128)
    x64 = x.astype(np.float64)
    logits = x64 @ L.router.astype(np.float64).T
    if L.router_bias is not None:
        logits += L.router_bias
    p = np.exp(logits - logits.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    n = x.shape[0]
    ids = np.empty((n, L.n_used), np.int64)
    for t in range(n):
        idx = np.arange(L.n_expert)
        key = idx if not tie_high else -idx
        order = np.lexsort((key, -p[t]))
        ids[t] = order[:L.n_used]
    w = np.take_along_axis(p, ids, axis=1)
    w = w / np.maximum(w.sum(axis=1, keepdims=True), 6.103515625e-5)
    out = np.zeros((n, L.E))
    cache = {}
    for t in range(n):
        xh = rotate64(x64[t], L.gate_signs, H)
        for k in range(L.n_used):
            e = int(ids[t, k])
            if swap_expert:
                e = (e + 1) % L.n_expert
            if e not in cache:
                cache[e] = [dense(oracle_mod, L, e, j) for j in range(3)]
            Wg, Wu, Wd = cache[e]
            g, u = Wg @ xh, Wu @ xh
            a = g / (1 + np.exp(-g)) * u
            if not drop_down_rotation:
                a = rotate64(a, L.down_signs, H)
            out[t] += w[t, k] * (Wd @ a)
    return out, ids, w


@pytest.fixture(scope="module")
def small_layer():
    return synth.make_layer(11, E=256, F=128, n_expert=16, n_used=4)


def test_layer_matches_numpy_fp64(oracle_mod, small_layer):
    L = small_layer
    x = synth.make_tokens(12, 6, L.E)
    ol = oracle_mod.OracleLayer(L)
    out, tr = ol.forward(x, threads=4, trace=True)
    ref, ids, w = numpy_layer(oracle_mod, L, x)
    np.testing.assert_array_equal(tr["route_ids"], ids)
    np.testing.assert_allclose(tr["route_w"], w, rtol=1e-5)
    assert oracle_mod.rel_rms(ref, out) < 1e-5
    assert oracle_mod.cosine(ref, out) > 0.999999
    # The oracle's own fp64 dense path agrees with numpy to rounding.
    d64 = ol.dense_f64(x, tr["route_ids"], tr["route_w"])
    assert oracle_mod.rel_rms(ref, d64) < 1e-6
    # The fp64 router logits (the margin guard's input) match numpy's x.W^T.
    r64 = ol.router_f64(x)
    np.testing.assert_allclose(r64, x.astype(np.float64) @ L.router.astype(np.float64).T, rtol=1e-12, atol=1e-12)
    # Planted mistakes fail.
    bad, _, _ = numpy_layer(oracle_mod, L, x, drop_down_rotation=True)
    assert oracle_mod.rel_rms(bad, out) > 0.1
    bad, _, _ = numpy_layer(oracle_mod, L, x, swap_expert=True)
    assert oracle_mod.rel_rms(bad, out) > 0.1


def test_layer_thread_count_invariant(oracle_mod, small_layer):
    """The pool decomposition (src/pool.zig:84-120) changes scheduling only, never results."""
    L = small_layer
    x = synth.make_tokens(13, 9, L.E)
    ol = oracle_mod.OracleLayer(L)
    a = ol.forward(x, threads=1)
    b = ol.forward(x, threads=7)
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))


def test_mixed_types_and_bias(oracle_mod):
    L = synth.make_layer(21, E=256, F=128, n_expert=16, n_used=4, mixed_types=True, zipf=1.1)
    assert len(np.unique(L.types)) > 4
    x = synth.make_tokens(22, 5, L.E)
    ol = oracle_mod.OracleLayer(L)
    out, tr = ol.forward(x, threads=3, trace=True)
    ref, ids, _ = numpy_layer(oracle_mod, L, x)
    np.testing.assert_array_equal(tr["route_ids"], ids)
    assert oracle_mod.rel_rms(ref, out) < 1e-5


def test_counting_sort_invariants(oracle_mod, small_layer):
    """src/engine.zig:553-564: a stable permutation of slots grouped by expert."""
    L = small_layer
    n = 40
    x = synth.make_tokens(14, n, L.E)
    _, tr = oracle_mod.OracleLayer(L).forward(x, threads=2, trace=True)
    ids = tr["route_ids"].reshape(-1)
    order, starts = tr["route_order"], tr["order_start"]
    assert sorted(order.tolist()) == list(range(n * L.n_used))
    assert starts[0] == 0 and starts[-1] == n * L.n_used
    for e in range(L.n_expert):
        seg = order[starts[e]:starts[e + 1]]
        assert np.all(ids[seg] == e)
        assert np.all(np.diff(seg.astype(np.int64)) > 0)
        assert len(seg) == int(np.sum(ids == e))


def test_topk_ties_and_brute_force(oracle_mod):
    """src/engine.zig:670-687: descending values, ties to the lower index."""
    g = np.random.default_rng(5)
    for trial in range(200):
        n = int(g.integers(8, 300))
        k = int(g.integers(1, 9))
        v = g.integers(0, 6, n).astype(np.float32) / 8  # many ties
        if trial % 3 == 0:
            v = g.standard_normal(n).astype(np.float32)
        ids, w = oracle_mod.topk(v, k)
        expect = np.lexsort((np.arange(n), -v))[:k]
        np.testing.assert_array_equal(ids, expect)
        np.testing.assert_array_equal(w, v[expect])
    # Planted mistake: preferring the higher index on ties disagrees.
    v = np.array([0.5, 0.5, 0.25], np.float32)
    ids, _ = oracle_mod.topk(v, 1)
    assert ids[0] == 0


def test_scale_zero_blocks_give_zero_output(oracle_mod):
    """Closed form: with every block scale zero, every expert decodes to zeros."""
    L = synth.make_layer(31, E=256, F=128, n_expert=8, n_used=2)
    for mats in (L.gate, L.up, L.down):
        for m in mats:
            v = m.reshape(m.shape[0], -1, 34)
            v[:, :, 0] = 0
            v[:, :, 1] = 0
    out = oracle_mod.OracleLayer(L).forward(synth.make_tokens(32, 3, L.E), threads=2)
    assert np.all(out == 0)


def bf16_to_f64(bits):
    return (np.asarray(bits, np.uint32) << 16).view(np.float32).astype(np.float64)


def shared_f64(L, which):
    """fp64 weights of a shared matrix in its GGML type: bf16 bits, Q8_0 rows (oracle decode,
    pinned on the reference's known answer in test_q8.py) or fp32 row bytes."""
    m = getattr(L, which)
    cols = L.SF if which == "sh_down" else L.E
    if L.sh_type == 30:
        return bf16_to_f64(m)
    if L.sh_type == 8:
        import oracle
        return oracle.q8_0_decode_rows(m, m.shape[0], cols).astype(np.float64)
    return np.ascontiguousarray(m).view(np.float32).reshape(m.shape[0], cols).astype(np.float64)


@pytest.mark.parametrize("sh_type", [30, 8, 0])
def test_shared_expert_matches_numpy(oracle_mod, sh_type):
    """The shared expert (src/engine.zig:644-653; dotRow of src/kernels.zig:201-210 for bf16,
    Q8_0 and fp32 rows): the difference it makes to the oracle's output equals an fp64 numpy model
    of sigmoid(g . x) * W_d (silu(W_g x) * W_u x) on the unrotated input."""
    L = synth.make_layer(71, E=256, F=128, n_expert=16, n_used=4, SF=64, sh_type=sh_type)
    x = synth.make_tokens(72, 5, L.E)
    with_sh = oracle_mod.OracleLayer(L).forward(x, threads=2)
    L0 = synth.make_layer(71, E=256, F=128, n_expert=16, n_used=4)
    without = oracle_mod.OracleLayer(L0).forward(x, threads=2)
    x64 = x.astype(np.float64)
    g = x64 @ shared_f64(L, "sh_gate").T
    u = x64 @ shared_f64(L, "sh_up").T
    a = g / (1 + np.exp(-g)) * u
    sh = a @ shared_f64(L, "sh_down").T
    gate = 1 / (1 + np.exp(-(x64 @ L.sh_gate_inp.astype(np.float64))))
    ref = gate[:, None] * sh
    got = with_sh.astype(np.float64) - without.astype(np.float64)
    assert oracle_mod.rel_rms(ref, got) < 1e-4
    # A planted mistake (gate = 1, the "always on" reading) fails.
    assert oracle_mod.rel_rms(sh, got) > 1e-2


def test_rms_norm_closed_forms(oracle_mod):
    """rmsNorm, src/kernels.zig:281-291: out = x / sqrt(mean(x^2) + eps) * w."""
    g = np.random.default_rng(81)
    n = 2048
    # A constant row c: mean square c^2, so out = sign(c) / sqrt(1 + eps / c^2) * w.
    for c, eps in ((3.0, 1e-6), (-0.25, 1e-2), (1e-3, 1e-6)):
        w = g.standard_normal(n).astype(np.float32)
        out = oracle_mod.rms_norm(np.full((1, n), c, np.float32), w, eps)[0]
        expect = np.sign(c) / np.sqrt(1 + eps / c ** 2) * w.astype(np.float64)
        np.testing.assert_allclose(out, expect, rtol=2e-6, atol=1e-7)
    # Unit mean square without weight at eps = 0, and invariance to a positive scale.
    x = g.standard_normal((4, n)).astype(np.float32)
    out = oracle_mod.rms_norm(x, None, 0.0)
    np.testing.assert_allclose(np.mean(out.astype(np.float64) ** 2, axis=1), 1.0, rtol=1e-5)
    np.testing.assert_allclose(oracle_mod.rms_norm(x * 8.0, None, 0.0), out, rtol=1e-5, atol=1e-6)
    # An fp64 numpy model with weight and eps.
    w = (1 + 0.1 * g.standard_normal(n)).astype(np.float32)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt(np.mean(x64 ** 2, axis=1, keepdims=True) + 1e-6) * w
    got = oracle_mod.rms_norm(x, w, 1e-6)
    assert oracle_mod.rel_rms(ref, got) < 1e-6
    # Planted mistakes fail: the sum in place of the mean, and a dropped weight.
    bad = x64 / np.sqrt(np.sum(x64 ** 2, axis=1, keepdims=True) + 1e-6) * w
    assert oracle_mod.rel_rms(bad, got) > 0.5
    bad = x64 / np.sqrt(np.mean(x64 ** 2, axis=1, keepdims=True) + 1e-6)
    assert oracle_mod.rel_rms(bad, got) > 0.05


def test_stack_matches_numpy(oracle_mod):
    """The residual stack x <- x + MoE_l(RMSNorm_l(x)) over three layers against the fp64 numpy
    model of each step; dropping the residual or the norm weight fails."""
    layers = synth.make_stack(91, 3, E=256, F=128, n_expert=16, n_used=4)
    x = synth.make_tokens(92, 3, 256)
    got = oracle_mod.stack_forward(layers, x, threads=2)
    ref = x.astype(np.float64)
    no_res = None
    for L in layers:
        h = ref / np.sqrt(np.mean(ref ** 2, axis=1, keepdims=True) + L.norm_eps) * L.norm_weight
        y, _, _ = numpy_layer(oracle_mod, L, h.astype(np.float32))
        if no_res is None:
            no_res = y
        ref = ref + y
    assert oracle_mod.rel_rms(ref, got) < 1e-5
    assert oracle_mod.rel_rms(no_res, got) > 0.1
