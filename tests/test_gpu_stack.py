"""GPU parity of the residual MoE stack x <- x + MoE_l(RMSNorm_l(x)) against the CPU oracle,
through the C ABI (gm_forward_stack, gm_run_stack).

Bar: final residual streams within relative RMS 2e-3 and cosine 0.9999 of the oracle's fp32
stack, per token. After the first layer the GPU's layer inputs differ from the oracle's by the
earlier layers' rounding, so a token whose 8th and 9th router probabilities lie within 3e-3
relative at any layer of the oracle's run may route differently; such tokens are reported and
excluded (the routing itself is bit-checked per layer by the single-layer tests). Stacks run
on the decode path (8 tokens), the prefill path (64 tokens), the reference path and the generic
path (mixed Gyro types with a shared expert); gm_run_stack over device-resident batches must
equal gm_forward_stack bit for bit.
"""
import numpy as np
import pytest

from gyrodx import synth
from gyrodx.engine import PATH_DECODE, PATH_GENERIC, PATH_PREFILL, PATH_REFERENCE, Engine

pytestmark = pytest.mark.gpu
REL_RMS = 2e-3
COSINE = 0.9999
MARGIN = 3e-3


def oracle_stack(oracle_mod, layers, x):
    """The oracle's stack and a mask of the tokens routed with a clear margin at every layer."""
    x = np.ascontiguousarray(x, np.float32).copy()
    clear = np.ones(x.shape[0], bool)
    for L in layers:
        ol = oracle_mod.OracleLayer(L)
        h = oracle_mod.rms_norm(x, L.norm_weight, L.norm_eps)
        logits = ol.router_f64(h)
        if L.router_bias is not None:
            logits = logits + L.router_bias.astype(np.float64)
        p = np.exp(logits - logits.max(axis=1, keepdims=True))
        s = -np.sort(-p, axis=1)
        U = L.n_used
        clear &= (s[:, U - 1] - s[:, U]) > MARGIN * s[:, U - 1]
        x = x + ol.forward(h)
    return x, clear


def check(oracle_mod, what, ref, out, clear, min_clear=0.6):
    n = ref.shape[0]
    print(f"{what}: {n - int(clear.sum())} of {n} tokens near a routing tie excluded", flush=True)
    assert clear.mean() >= min_clear, (what, int(clear.sum()))
    r = oracle_mod.rel_rms(ref[clear], out[clear])
    c = oracle_mod.cosine(ref[clear], out[clear])
    worst = max(oracle_mod.rel_rms(ref[t], out[t]) for t in np.flatnonzero(clear))
    print(f"{what}: rel_rms={r:.3e} worst token={worst:.3e} cosine={c:.8f}", flush=True)
    assert r <= REL_RMS and worst <= 2 * REL_RMS and c >= COSINE, (what, r, worst, c)


@pytest.fixture(scope="module")
def full_stack():
    return synth.make_stack(4801, 4)


def make_engine(layers, max_tok):
    eng = Engine(max_tok=max_tok)
    ids = [eng.add_layer(L) for L in layers]
    return eng, ids


def test_stack_decode_path(oracle_mod, full_stack):
    x = synth.make_tokens(4802, 8)
    ref, clear = oracle_stack(oracle_mod, full_stack, x)
    eng, ids = make_engine(full_stack, 8)
    try:
        print("stack decode: 4 layers, 8 tokens", flush=True)
        out = eng.forward_stack(ids, x, PATH_DECODE)
        check(oracle_mod, "stack decode", ref, out, clear, min_clear=0.5)
        # A single token as well.
        ref1, clear1 = oracle_stack(oracle_mod, full_stack, x[3:4])
        out1 = eng.forward_stack(ids, x[3:4], PATH_DECODE)
        if clear1[0]:
            check(oracle_mod, "stack decode n=1", ref1, out1, clear1)
    finally:
        eng.close()


def test_stack_prefill_path_and_run(oracle_mod, full_stack):
    x = synth.make_tokens(4803, 64, bf16=True)
    ref, clear = oracle_stack(oracle_mod, full_stack, x)
    eng, ids = make_engine(full_stack, 64)
    try:
        print("stack prefill: 4 layers, 64 tokens", flush=True)
        out = eng.forward_stack(ids, x, PATH_PREFILL)
        check(oracle_mod, "stack prefill", ref, out, clear)
        # Device-resident batches through gm_run_stack: two calls of 32 tokens equal
        # gm_forward_stack on each batch.
        eng.set_tokens(x)
        print("stack prefill: gm_run_stack 2 x 32", flush=True)
        dev_ms, wall_ms = eng.run_stack(PATH_PREFILL, 32, 2, ids)
        assert dev_ms > 0 and wall_ms > 0
        got = eng.read_outputs(64)
        for b in range(2):
            one = eng.forward_stack(ids, x[32 * b:32 * (b + 1)], PATH_PREFILL)
            np.testing.assert_array_equal(got[32 * b:32 * (b + 1)].view(np.uint32), one.view(np.uint32))
    finally:
        eng.close()


def test_stack_coder_shapes_decode_and_prefill(oracle_mod):
    """Three layers at the real model's expert shapes (hidden 2560, F 640, top-10) through the
    decode path (moe_decode_gu_g / moe_decode_down_g, 6 tokens) and the prefill path (48)."""
    layers = synth.make_stack(4841, 3, E=2560, F=640, n_expert=128, n_used=10)
    eng, ids = make_engine(layers, 48)
    try:
        for path, n, name in ((PATH_DECODE, 6, "decode"), (PATH_PREFILL, 48, "prefill")):
            x = synth.make_tokens(4842 + n, n, 2560, bf16=True)
            ref, clear = oracle_stack(oracle_mod, layers, x)
            print(f"stack coder shapes {name}: 3 layers, {n} tokens", flush=True)
            out = eng.forward_stack(ids, x, path)
            check(oracle_mod, f"stack coder shapes {name}", ref, out, clear, min_clear=0.5)
    finally:
        eng.close()


def test_stack_reference_path(oracle_mod):
    layers = synth.make_stack(4811, 3, E=1024, F=256, n_expert=64, n_used=4)
    layers[1].norm_weight = None  # a layer without norm weight
    x = synth.make_tokens(4812, 5, 1024)
    ref, clear = oracle_stack(oracle_mod, layers, x)
    eng, ids = make_engine(layers, 8)
    try:
        print("stack reference: 3 layers, 5 tokens", flush=True)
        out = eng.forward_stack(ids, x, PATH_REFERENCE)
        check(oracle_mod, "stack reference", ref, out, clear, min_clear=0.4)
    finally:
        eng.close()


def test_stack_generic_path_mixed_shared(oracle_mod):
    layers = synth.make_stack(4821, 2, E=1024, F=256, n_expert=32, n_used=4, mixed_types=True, SF=128)
    x = synth.make_tokens(4822, 6, 1024)
    ref, clear = oracle_stack(oracle_mod, layers, x)
    eng, ids = make_engine(layers, 8)
    try:
        print("stack generic: 2 mixed layers with shared expert, 6 tokens", flush=True)
        out = eng.forward_stack(ids, x, PATH_GENERIC)
        check(oracle_mod, "stack generic", ref, out, clear, min_clear=0.4)
    finally:
        eng.close()


def test_stack_rejects_bad_layer_list():
    layers = synth.make_stack(4831, 1, E=256, F=128, n_expert=8, n_used=2)
    eng, ids = make_engine(layers, 4)
    try:
        x = synth.make_tokens(4832, 2, 256)
        with pytest.raises(RuntimeError):
            eng.forward_stack([5], x, PATH_REFERENCE)
        with pytest.raises(RuntimeError):
            eng.forward_stack([], x, PATH_REFERENCE)
    finally:
        eng.close()


STACK_NORM_CASES = [
    # layers, E, F, experts, top-k, tokens, make_stack extras, layer without a norm weight
    (4, 2048, 512, 256, 8, 64, {}, 2),
    (3, 4096, 256, 32, 4, 33, {}, None),
    (3, 1024, 512, 64, 8, 40, {"SF": 256}, 1),
    (2, 2560, 640, 64, 10, 17, {}, None),
]


@pytest.mark.parametrize("nl,E,F,NE,U,n,kw,bare", STACK_NORM_CASES,
                         ids=[f"{c[0]}x-E{c[1]}-F{c[2]}-x{c[3]}-top{c[4]}-n{c[5]}" + "".join(f"-{k}" for k in c[6])
                              for c in STACK_NORM_CASES])
def test_stack_prefill_fused_norm(oracle_mod, monkeypatch, nl, E, F, NE, U, n, kw, bare):
    """On the prefill path every layer's combine but the last also writes the next layer's
    RMSNorm (moe_prefill_combine_norm), so only the first layer runs moe_stack_norm. The final
    stream must equal, bit for bit, the one of an engine created with GYRO_STACK_NORM_FUSED=0
    (moe_stack_norm before every layer), with a bf16 shared expert (its gate dot reads the
    normalised rows the kernel overwrites), a layer without a norm weight and hidden sizes up to
    4096; gm_run_stack equals gm_forward_stack; the stream is within the oracle's bar."""
    layers = synth.make_stack(4860 + E // 256 + n, nl, E=E, F=F, n_expert=NE, n_used=U, **kw)
    if bare is not None:
        layers[bare].norm_weight = None
    x = synth.make_tokens(4861 + n, n, E)
    outs = {}
    for fused in ("1", "0"):
        monkeypatch.setenv("GYRO_STACK_NORM_FUSED", fused)
        eng, ids = make_engine(layers, n)
        try:
            print(f"prefill stack {nl} layers E={E} F={F} experts={NE} top-{U} n={n} {kw} fused norm {fused}",
                  flush=True)
            outs[fused] = eng.forward_stack(ids, x, PATH_PREFILL)
            if fused == "1":
                eng.set_tokens(x)
                eng.run_stack(PATH_PREFILL, n, 1, ids)
                np.testing.assert_array_equal(eng.read_outputs(n).view(np.uint32), outs[fused].view(np.uint32))
        finally:
            eng.close()
    np.testing.assert_array_equal(outs["1"].view(np.uint32), outs["0"].view(np.uint32))
    ref, clear = oracle_stack(oracle_mod, layers, x)
    check(oracle_mod, f"fused-norm prefill stack E={E}", ref, outs["1"], clear, min_clear=0.3)
