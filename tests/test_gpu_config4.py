"""GPU parity of the 48-layer resident stack (hidden 2048, 256 experts, top-8, F 512, TQ2_T;
48 x 256 bundles = 10,267,656,192 bytes) through the C ABI.

The bundles fill 2 GiB arenas of 2,570 slots (src/gpu_engine.zig:593-650); a layer's 256
bundles never straddle two arenas, so ten layers share an arena and the stack spans five: every
layer past the tenth is addressed through an arena index > 0 (moe_resolve on the reference path,
base + e * slot_stride on the fast paths).

A free-running 48-layer comparison would exclude most tokens (each layer adds a chance of a
near-tie in the top-8), so each layer is checked teacher-forced: it receives the oracle's
residual stream x_l, the stack path computes x_l + MoE_l(RMSNorm_l(x_l)) through gm_forward_stack
on that one layer, and its MoE contribution is compared with the oracle's to rel-RMS 2e-3 and
cosine 0.9999 over the tokens whose routing at that layer is separable (8th/9th fp64 probability
gap above 1e-5 relative). Decode at batch 1 and 8, prefill at batch 32 (the small-tile GEMM
launch) and 64; gm_run_stack over all 48 layers equals gm_forward_stack bit for bit.

The sweep's 4096-token prefill (32,768 slots per layer, the largest call) is checked on the GPU's
own stream: one gm_forward_stack over all 48 layers must equal the 48 one-layer calls chained on
the GPU's outputs bit for bit, and at every layer the MoE contribution of 64 sampled tokens must
match the oracle's layer computed from that same stream (the oracle on all 4096 tokens x 48 layers
would take minutes; each token's result depends on its own row only).
"""
import numpy as np
import pytest

from gyrodx import synth
from gyrodx.engine import PATH_DECODE, PATH_PREFILL, PATH_REFERENCE, Engine

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(900)]
N_LAYERS = 48


@pytest.fixture(scope="module")
def stack48():
    print("config 4: generating 48 layers", flush=True)
    layers = synth.make_stack(4900, N_LAYERS)
    eng = Engine(max_tok=4096)
    print("config 4: uploading 10.27 GB of experts", flush=True)
    ids = [eng.add_layer(L) for L in layers]
    assert ids == list(range(N_LAYERS))
    yield layers, eng
    eng.close()


def oracle_streams(oracle_mod, layers, x):
    """The oracle's residual stream before each layer and each layer's MoE output."""
    xs, moe = [], []
    x = np.ascontiguousarray(x, np.float32).copy()
    for L in layers:
        xs.append(x.copy())
        h = oracle_mod.rms_norm(x, L.norm_weight, L.norm_eps)
        y = oracle_mod.OracleLayer(L).forward(h)
        moe.append(y)
        x = x + y
    return xs, moe


def separable(oracle_mod, L, x, margin=1e-5):
    h = oracle_mod.rms_norm(x, L.norm_weight, L.norm_eps)
    logits = oracle_mod.OracleLayer(L).router_f64(h)
    p = np.exp(logits - logits.max(axis=1, keepdims=True))
    s = -np.sort(-p, axis=1)
    return (s[:, L.n_used - 1] - s[:, L.n_used]) > margin * s[:, L.n_used - 1]


def teacher_forced(oracle_mod, layers, eng, path, n, seed, what):
    x = synth.make_tokens(seed, n, bf16=path == PATH_PREFILL)
    xs, moe = oracle_streams(oracle_mod, layers, x)
    worst_r, worst_c, excluded = 0.0, 1.0, 0
    for l, L in enumerate(layers):
        got = eng.forward_stack([l], xs[l], path).astype(np.float64) - xs[l].astype(np.float64)
        sep = separable(oracle_mod, L, xs[l])
        excluded += int((~sep).sum())
        r = oracle_mod.rel_rms(moe[l][sep], got[sep])
        c = oracle_mod.cosine(moe[l][sep], got[sep])
        worst_r, worst_c = max(worst_r, r), min(worst_c, c)
        assert r <= 2e-3 and c >= 0.9999, (what, l, r, c)
    print(f"{what}: 48 layers teacher-forced, worst rel_rms={worst_r:.3e} worst cosine={worst_c:.8f}, "
          f"{excluded} token-layers near a routing tie excluded", flush=True)


def test_stack48_decode_batch1_and_8(oracle_mod, stack48):
    layers, eng = stack48
    teacher_forced(oracle_mod, layers, eng, PATH_DECODE, 1, 4901, "stack48 decode n=1")
    teacher_forced(oracle_mod, layers, eng, PATH_DECODE, 8, 4902, "stack48 decode n=8")


def test_stack48_prefill_batch64(oracle_mod, stack48):
    layers, eng = stack48
    teacher_forced(oracle_mod, layers, eng, PATH_PREFILL, 64, 4903, "stack48 prefill n=64")


def test_stack48_prefill_batch32(oracle_mod, stack48):
    layers, eng = stack48
    teacher_forced(oracle_mod, layers, eng, PATH_PREFILL, 32, 4905, "stack48 prefill n=32")


def test_stack48_prefill_4096(oracle_mod, stack48):
    layers, eng = stack48
    n = 4096
    x = synth.make_tokens(4906, n, bf16=True)
    print("stack48 prefill n=4096: one call over 48 layers", flush=True)
    full = eng.forward_stack(list(range(N_LAYERS)), x, PATH_PREFILL)
    idx = np.arange(0, n, n // 64)
    cur = np.ascontiguousarray(x, np.float32)
    worst_r, worst_c, excluded = 0.0, 1.0, 0
    for l, L in enumerate(layers):
        nxt = eng.forward_stack([l], cur, PATH_PREFILL)
        xs = cur[idx]
        got = nxt[idx].astype(np.float64) - xs.astype(np.float64)
        ref = oracle_mod.OracleLayer(L).forward(oracle_mod.rms_norm(xs, L.norm_weight, L.norm_eps))
        sep = separable(oracle_mod, L, xs)
        excluded += int((~sep).sum())
        r, c = oracle_mod.rel_rms(ref[sep], got[sep]), oracle_mod.cosine(ref[sep], got[sep])
        worst_r, worst_c = max(worst_r, r), min(worst_c, c)
        assert r <= 2e-3 and c >= 0.9999, ("stack48 prefill n=4096", l, r, c)
        cur = nxt
    np.testing.assert_array_equal(full.view(np.uint32), cur.view(np.uint32))
    print(f"stack48 prefill n=4096: one call equals 48 chained calls; 64 sampled tokens per layer, worst "
          f"rel_rms={worst_r:.3e} worst cosine={worst_c:.8f}, {excluded} token-layers near a routing tie "
          f"excluded", flush=True)


def test_stack48_reference_path_far_arena(oracle_mod, stack48):
    """The reference dispatch (moe_resolve's arena lookup) on the last layer, in arena 4."""
    layers, eng = stack48
    x = synth.make_tokens(4904, 4)
    xs, moe = oracle_streams(oracle_mod, layers[-1:], x)
    got = eng.forward_stack([N_LAYERS - 1], xs[0], PATH_REFERENCE).astype(np.float64) - xs[0]
    sep = separable(oracle_mod, layers[-1], xs[0])
    r, c = oracle_mod.rel_rms(moe[0][sep], got[sep]), oracle_mod.cosine(moe[0][sep], got[sep])
    print(f"stack48 reference path, layer 47: rel_rms={r:.3e} cosine={c:.8f}", flush=True)
    assert r <= 2e-3 and c >= 0.9999


def test_stack48_run_equals_forward(stack48):
    """gm_run_stack (the benchmark harness) over all 48 layers equals gm_forward_stack."""
    layers, eng = stack48
    x = synth.make_tokens(4905, 16)
    eng.set_tokens(x)
    ids = list(range(N_LAYERS))
    for path, batch in ((PATH_DECODE, 8), (PATH_PREFILL, 16)):
        eng.run_stack(path, batch, 16 // batch, ids)
        got = eng.read_outputs(16)
        for b in range(16 // batch):
            one = eng.forward_stack(ids, x[b * batch:(b + 1) * batch], path)
            np.testing.assert_array_equal(got[b * batch:(b + 1) * batch].view(np.uint32), one.view(np.uint32))
        print(f"stack48 gm_run_stack path {path} batch {batch}: equal to gm_forward_stack", flush=True)
