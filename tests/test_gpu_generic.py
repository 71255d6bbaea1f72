"""GPU parity of the generic path (mixed Gyro types per expert and projection, bf16 shared
expert) and of the reference path with a shared expert, against the CPU oracle, through the C
ABI. Bar as in test_gpu_moe.py: top-k ids identical for separable tokens, rel-RMS <= 2e-3,
cosine >= 0.9999."""
import numpy as np
import pytest

from gyrodx import synth
from gyrodx.engine import PATH_GENERIC, PATH_REFERENCE, Engine

pytestmark = pytest.mark.gpu


def separable(oracle_layer, x, U, margin=1e-5):
    logits = oracle_layer.router_f64(x)
    if oracle_layer.layer.router_bias is not None:
        logits = logits + oracle_layer.layer.router_bias.astype(np.float64)
    p = np.exp(logits - logits.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    s = -np.sort(-p, axis=1)
    return (s[:, U - 1] - s[:, U]) > margin * s[:, U - 1]


def check(oracle_mod, layer, x, path, what, max_tok=16):
    eng = Engine(max_tok=max(max_tok, x.shape[0]))
    try:
        eng.add_layer(layer)
        ol = oracle_mod.OracleLayer(layer)
        ref, tr = ol.forward(x, trace=True)
        print(f"{what}: n={x.shape[0]} types={sorted(set(layer.types.ravel().tolist()))} SF={layer.SF}", flush=True)
        out = eng.forward(0, x, path)
        ids, _ = eng.last_routes(x.shape[0])
        sep = separable(ol, x, layer.n_used)
        np.testing.assert_array_equal(ids[sep], tr["route_ids"][sep])
        r, c = oracle_mod.rel_rms(ref, out), oracle_mod.cosine(ref, out)
        print(f"{what}: rel_rms={r:.3e} cosine={c:.8f} excluded={int((~sep).sum())}", flush=True)
        assert r <= 2e-3 and c >= 0.9999, (what, r, c)
    finally:
        eng.close()


def test_generic_mixed_types_small(oracle_mod):
    layer = synth.make_layer(81, E=1024, F=256, n_expert=32, n_used=8, mixed_types=True)
    assert len(np.unique(layer.types)) == 8
    check(oracle_mod, layer, synth.make_tokens(82, 11, layer.E), PATH_GENERIC, "mixed small")


def test_generic_mixed_quant_layer_with_shared_expert(oracle_mod):
    """The mixed-quant configuration: hidden 2048, 256 experts, top-8, F 512, all eight Gyro types
    assigned by seed per expert and projection, a bf16 shared expert of width 1024, rotations."""
    layer = synth.make_layer(91, mixed_types=True, SF=1024)
    check(oracle_mod, layer, synth.make_tokens(92, 4, layer.E), PATH_GENERIC, "mixed quant + shared")


def test_reference_path_with_shared_expert(oracle_mod):
    layer = synth.make_layer(101, E=1024, F=256, n_expert=32, n_used=8, SF=256)
    check(oracle_mod, layer, synth.make_tokens(102, 9, layer.E), PATH_REFERENCE, "reference + shared")
    check(oracle_mod, layer, synth.make_tokens(103, 9, layer.E), PATH_GENERIC, "generic + shared")


def test_decode_path_mixed_quant_and_shared(oracle_mod):
    """The decode path's type-generic kernels (moe_decode_gu_x, moe_decode_down_x) on the
    mixed-quant configuration, with and without the shared expert, at batch 1 and 8."""
    from gyrodx.engine import PATH_DECODE
    mixed = synth.make_layer(111, mixed_types=True)
    check(oracle_mod, mixed, synth.make_tokens(112, 1, mixed.E), PATH_DECODE, "decode mixed n=1")
    check(oracle_mod, mixed, synth.make_tokens(113, 8, mixed.E), PATH_DECODE, "decode mixed n=8")
    shared = synth.make_layer(91, mixed_types=True, SF=1024)
    check(oracle_mod, shared, synth.make_tokens(114, 1, shared.E), PATH_DECODE, "decode mixed + shared n=1")
    check(oracle_mod, shared, synth.make_tokens(115, 5, shared.E), PATH_DECODE, "decode mixed + shared n=5")


def test_decode_path_mixed_hidden_1024(oracle_mod):
    """The same kernels at hidden 1024 (E / 8 = 128 down groups for one token, 8 rows each;
    E / 16 per token for 2 to 8 tokens), with a shared expert of width 256 and without."""
    from gyrodx.engine import PATH_DECODE
    for seed, SF in ((121, 0), (123, 256)):
        layer = synth.make_layer(seed, E=1024, F=512, n_expert=64, n_used=8, mixed_types=True, SF=SF)
        for n in (1, 3, 8):
            check(oracle_mod, layer, synth.make_tokens(seed + n, n, layer.E), PATH_DECODE,
                  f"decode mixed E=1024 SF={SF} n={n}")


@pytest.mark.parametrize("type_id", [145, 147, 149, 151])
def test_decode_path_uniform_other_types(oracle_mod, type_id):
    """Uniform non-TQ2_T layers (32- and 64-step trellises) through the type-generic decode."""
    from gyrodx.engine import PATH_DECODE
    layer = synth.make_layer(120 + type_id, type_id=type_id)
    check(oracle_mod, layer, synth.make_tokens(121 + type_id, 3, layer.E), PATH_DECODE, f"decode type {type_id}")


def test_prefill_path_mixed_types(oracle_mod):
    """The type-generic grouped GEMMs (moe_prefill_gu_x, moe_prefill_down_x) on the mixed-quant
    layer: a Gyro type per expert and projection drawn from all eight, rotations; 512 tokens and
    a ragged 37."""
    from gyrodx.engine import PATH_PREFILL
    layer = synth.make_layer(131, mixed_types=True)
    check(oracle_mod, layer, synth.make_tokens(132, 512, layer.E), PATH_PREFILL, "prefill mixed n=512")
    check(oracle_mod, layer, synth.make_tokens(133, 37, layer.E), PATH_PREFILL, "prefill mixed n=37")


@pytest.mark.parametrize("type_id", [145, 147, 149, 151])
def test_prefill_path_uniform_other_types(oracle_mod, type_id):
    """Uniform non-TQ2_T layers (32- and 64-step trellises, 18- to 58-byte blocks) through the
    type-generic prefill GEMMs, without rotations for one of them."""
    from gyrodx.engine import PATH_PREFILL
    layer = synth.make_layer(140 + type_id, type_id=type_id, signs=type_id != 147)
    check(oracle_mod, layer, synth.make_tokens(141 + type_id, 200, layer.E), PATH_PREFILL, f"prefill type {type_id}")


@pytest.mark.parametrize("type_id,E,F,NE,U", [(148, 2560, 640, 64, 10), (0, 1024, 384, 64, 6)])
def test_prefill_path_generic_types_odd_down_blocks(oracle_mod, type_id, E, F, NE, U):
    """The type-generic prefill GEMMs with an odd block count per down row (F 640 and 384: odd
    rows start 2 bytes off a 4-byte boundary) and other top-k widths: a uniform 64-step type at
    the real model's hidden 2560 / F 640 / top-10, and mixed types (type_id 0) at F 384, top-6."""
    from gyrodx.engine import PATH_PREFILL
    kw = dict(mixed_types=True) if type_id == 0 else dict(type_id=type_id)
    layer = synth.make_layer(160 + U, E=E, F=F, n_expert=NE, n_used=U, **kw)
    check(oracle_mod, layer, synth.make_tokens(161 + U, 90, layer.E), PATH_PREFILL,
          f"prefill type {type_id or 'mixed'} E={E} F={F} top-{U}")


@pytest.mark.parametrize("type_id,E,F,NE,U", [(148, 2560, 640, 64, 10), (0, 1024, 384, 64, 6),
                                               (151, 1280, 1024, 48, 16)])
def test_decode_path_generic_types_other_shapes(oracle_mod, type_id, E, F, NE, U):
    """The general type-generic decode (moe_decode_gu_xg, moe_decode_down_xg): hidden 2560 and
    1280, odd block counts per down row (F 640, 384), F 1024, top-k widths 6, 10 and 16, one
    type or all eight mixed per expert and projection (both half-block stream rotations: word
    and half-word), at 1, 3 and 8 tokens."""
    from gyrodx.engine import PATH_DECODE
    kw = dict(mixed_types=True) if type_id == 0 else dict(type_id=type_id)
    layer = synth.make_layer(170 + U, E=E, F=F, n_expert=NE, n_used=U, **kw)
    for n in (1, 3, 8):
        check(oracle_mod, layer, synth.make_tokens(171 + U + n, n, layer.E), PATH_DECODE,
              f"decode type {type_id or 'mixed'} E={E} F={F} top-{U}")


def test_prefill_falls_back_on_fp16_overflowing_scales_any_type(oracle_mod):
    """A block scale of any Gyro type whose products with the codebook overflow binary16 (scale
    60000 in one down block of expert 3 of a mixed-type layer) keeps the layer off the fp16
    grouped GEMMs: prefill calls run on the generic path's fp32 kernels, against the oracle."""
    from gyrodx.engine import PATH_PREFILL
    layer = synth.make_layer(151, E=1024, F=256, n_expert=16, n_used=8, mixed_types=True)
    e = 3
    layer.down[e][7, 0:2] = np.frombuffer(np.float16(60000.0).tobytes(), np.uint8)
    x = synth.make_tokens(152, 16, layer.E)
    ref = oracle_mod.OracleLayer(layer).forward(x)
    eng = Engine(max_tok=16)
    try:
        eng.add_layer(layer)
        out = eng.forward(0, x, PATH_PREFILL)
        ids, _ = eng.last_routes(16)
        assert (ids == e).any(), "no token routed to the outlier expert"
        r, c = oracle_mod.rel_rms(ref, out), oracle_mod.cosine(ref, out)
        print(f"mixed-type prefill with an overflowing block scale: rel_rms {r:.3e} cosine {c:.8f}", flush=True)
        assert r <= 2e-3 and c >= 0.9999
    finally:
        eng.close()


def test_prefill_path_with_shared_expert(oracle_mod):
    """The prefill path's shared expert (moe_prefill_shared gate/up and down on binary16 copies of
    the bf16 weights, the gate dot in moe_prefill_combine) on the mixed-quant configuration (SF
    1024) at 512 tokens and a ragged 37, and on a uniform TQ2_T layer with SF 256."""
    from gyrodx.engine import PATH_PREFILL
    mixed = synth.make_layer(91, mixed_types=True, SF=1024)
    check(oracle_mod, mixed, synth.make_tokens(161, 512, mixed.E), PATH_PREFILL, "prefill mixed + shared n=512")
    check(oracle_mod, mixed, synth.make_tokens(162, 37, mixed.E), PATH_PREFILL, "prefill mixed + shared n=37")
    tq2 = synth.make_layer(163, E=1024, F=256, n_expert=32, n_used=8, SF=256)
    check(oracle_mod, tq2, synth.make_tokens(164, 100, tq2.E), PATH_PREFILL, "prefill TQ2_T + shared n=100")
