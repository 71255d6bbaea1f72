"""The split-binary16 arithmetic of the prefill router (moe_prefill_router), restated in numpy.

The kernel computes logits[t][r] = W[r] . x[t] (src/engine.zig:526, an fp32 matmul) on binary16
MFMA: every fp32 value v is carried as hi = f16(v) and lo = f16((v - hi) 2^11), the router rows
scaled per row by 2^k_r at load time, and the products hi_x hi_w + 2^-11 (hi_x lo_w + lo_x hi_w)
accumulate in fp32. These checks run on the CPU: the layout that the engine and the integration
snippet share, the reconstruction error of the split (2^-22 relative), and the logit error
against fp64, with the plausible mistakes (the cross products dropped, the 2^11 or 2^-k_r
scale forgotten, lo_w and lo_x swapped for hi) shown to fail the same bound.
"""
import numpy as np

from test_integration_snippets import split_router_rows


def unpack(words: np.ndarray, NE: int, E: int):
    h = words[:NE * E].view(np.float16).reshape(NE, E // 16, 2, 16)
    hi = h[:, :, 0, :].reshape(NE, E).astype(np.float64)
    lo = h[:, :, 1, :].reshape(NE, E).astype(np.float64)
    unscale = words[NE * E:].view(np.float32).astype(np.float64)
    return hi, lo, unscale


def split_tokens(x: np.ndarray):
    hi = x.astype(np.float16)
    lo = ((x.astype(np.float32) * np.float32(2048)) - hi.astype(np.float32) * np.float32(2048)).astype(np.float16)
    return hi.astype(np.float64), lo.astype(np.float64)


def logits_split(x, words, NE, E, cross=True, two11=2048.0, use_unscale=True):
    wh, wl, unscale = unpack(words, NE, E)
    xh, xl = split_tokens(x)
    acc = xh @ wh.T
    if cross:
        acc = acc + (xh @ wl.T + xl @ wh.T) / two11
    return acc * (unscale[None, :] if use_unscale else 1.0)


def layer(seed, NE=32, E=512, n=24, wscale=0.02):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((NE, E)) * wscale).astype(np.float32)
    w[3] *= 1e-3  # a row far below the others: its own scale keeps its precision
    w[5, 7] = 0.0
    x = rng.standard_normal((n, E)).astype(np.float32)
    x[2] *= 1e-3  # small activations: lo stays normal through the 2^11 factor
    x[4, :8] = 3000.0
    return w, x


def test_layout_and_scales():
    w, _ = layer(1)
    NE, E = w.shape
    words = split_router_rows(w)
    assert words.dtype == np.uint32 and words.size == NE * E + NE
    hi, lo, unscale = unpack(words, NE, E)
    k = -np.log2(unscale)
    assert np.all(k == np.round(k))
    scaled = np.abs(hi).max(axis=1)
    assert np.all((scaled >= 2.0 ** 14) & (scaled <= 2.0 ** 15))
    # Row 0, chunk 1 (k = 16 .. 31): words 16 .. 23 hold the hi values, 24 .. 31 the lo values.
    first = words[16:32].view(np.float16).astype(np.float64)
    np.testing.assert_array_equal(first[:16], hi[0, 16:32])
    np.testing.assert_array_equal(first[16:], lo[0, 16:32])


def test_reconstruction_22_bits():
    w, x = layer(2)
    NE, E = w.shape
    hi, lo, unscale = unpack(split_router_rows(w), NE, E)
    rec = (hi + lo / 2048.0) * unscale[:, None]
    err = np.abs(rec - w.astype(np.float64))
    assert np.all(err <= 2.0 ** -22 * np.abs(w) + 1e-30)
    assert np.all(rec[w == 0] == 0)
    xh, xl = split_tokens(x)
    recx = xh + xl / 2048.0
    assert np.all(np.abs(recx - x) <= 2.0 ** -22 * np.abs(x) + 2.0 ** -36)


def test_logits_against_fp64_and_mistakes():
    w, x = layer(3)
    NE, E = w.shape
    words = split_router_rows(w)
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    bound = 2.0 ** -20 * (np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64).T)
    good = logits_split(x, words, NE, E)
    assert np.all(np.abs(good - exact) <= bound)
    # fp32 products summed in fp32 (the old fp32 MFMA's arithmetic) land in the same bound.
    f32 = (x @ w.T).astype(np.float64)
    assert np.all(np.abs(f32 - exact) <= bound)
    for bad in (dict(cross=False), dict(two11=1.0), dict(use_unscale=False)):
        assert np.any(np.abs(logits_split(x, words, NE, E, **bad) - exact) > bound), bad
    # The lo halves taken for the hi halves: the layout matters.
    swapped = words.copy()
    h = swapped[:NE * E].view(np.uint16).reshape(NE, E // 16, 2, 16)
    h[:, :, [0, 1], :] = h[:, :, [1, 0], :]
    assert np.any(np.abs(logits_split(x, swapped, NE, E) - exact) > bound)


def test_topk_unchanged_on_separable_tokens():
    """Top-8 of the split logits equals fp64's wherever the 8th and 9th fp64 logits differ by
    more than the error bound (the parity tests' near-tie rule is stricter)."""
    w, x = layer(4, NE=256, E=2048, n=64, wscale=0.01)
    words = split_router_rows(w)
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    got = logits_split(x, words, 256, 2048)
    order = np.argsort(-exact, axis=1, kind="stable")
    s = np.take_along_axis(exact, order, axis=1)
    sep = (s[:, 7] - s[:, 8]) > 1e-5 * np.abs(s[:, 7])
    assert sep.sum() >= 60
    mine = np.argsort(-got, axis=1, kind="stable")[:, :8]
    np.testing.assert_array_equal(np.sort(mine[sep], axis=1), np.sort(order[sep, :8], axis=1))
