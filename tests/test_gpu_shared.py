"""GPU parity of the shared expert in each row format the reference's GPU path binds
(src/gpu_engine.zig:289-306 and :846-851: Q8_0 repacked for mv_q8, bf16, fp32) against the CPU
oracle (dotRow of src/kernels.zig:201-210), through the C ABI, at the real model's shapes:
hidden 2560, F 640, top-10, a shared expert of width 640 (docs/MODEL.md:60-67). The decode path
runs such a shared expert in the mv kernels ahead of the routed kernels; the prefill path in its
binary16 GEMMs. Bar as in test_gpu_moe.py: top-k ids identical for separable tokens,
rel-RMS <= 2e-3, cosine >= 0.9999."""
import numpy as np
import pytest

from gyrodx import synth
from gyrodx.engine import PATH_DECODE, PATH_GENERIC, PATH_PREFILL, PATH_REFERENCE, Engine
from test_gpu_generic import check
from test_gpu_stack import check as check_stack, oracle_stack

pytestmark = pytest.mark.gpu

CODER = dict(E=2560, F=640, n_expert=64, n_used=10)


@pytest.mark.parametrize("sh_type", [8, 30, 0])
def test_coder_shape_shared_expert_decode(oracle_mod, sh_type):
    layer = synth.make_layer(601 + sh_type, SF=640, sh_type=sh_type, **CODER)
    for n in (1, 3, 8):
        check(oracle_mod, layer, synth.make_tokens(611 + n, n, layer.E), PATH_DECODE,
              f"decode shared type {sh_type} n={n}")


@pytest.mark.parametrize("sh_type", [8, 30, 0])
def test_coder_shape_shared_expert_prefill(oracle_mod, sh_type):
    layer = synth.make_layer(621 + sh_type, SF=640, sh_type=sh_type, **CODER)
    check(oracle_mod, layer, synth.make_tokens(631, 96, layer.E, bf16=True), PATH_PREFILL,
          f"prefill shared type {sh_type}", max_tok=96)


def test_q8_shared_expert_reference_and_generic_paths(oracle_mod):
    layer = synth.make_layer(641, SF=640, sh_type=8, **CODER)
    check(oracle_mod, layer, synth.make_tokens(642, 5, layer.E), PATH_REFERENCE, "reference q8 shared")
    check(oracle_mod, layer, synth.make_tokens(643, 5, layer.E), PATH_GENERIC, "generic q8 shared")


def test_q8_shared_expert_at_the_tuned_decode_shape(oracle_mod):
    """Hidden 2048, F 512, top-8 with a Q8_0 shared expert: the TQ2_T decode kernels plus the
    shared expert as the down kernel's residual input; also a mixed-type layer (the _x kernels)."""
    layer = synth.make_layer(651, E=2048, F=512, n_expert=64, n_used=8, SF=1024, sh_type=8)
    check(oracle_mod, layer, synth.make_tokens(652, 2, layer.E), PATH_DECODE, "decode tuned q8 shared")
    mixed = synth.make_layer(653, E=2048, F=512, n_expert=64, n_used=8, SF=512, sh_type=8, mixed_types=True)
    check(oracle_mod, mixed, synth.make_tokens(654, 4, mixed.E), PATH_DECODE, "decode mixed q8 shared")


@pytest.mark.parametrize("path", [PATH_DECODE, PATH_PREFILL])
def test_stack_with_q8_shared_expert(oracle_mod, path):
    """Two layers of x <- x + MoE(RMSNorm(x)) with Q8_0 shared experts, against the oracle stack."""
    layers = synth.make_stack(661, 2, SF=640, sh_type=8, **CODER)
    n = 4 if path == PATH_DECODE else 40
    x = synth.make_tokens(662, n, layers[0].E, bf16=path == PATH_PREFILL)
    eng = Engine(max_tok=n)
    try:
        ids = [eng.add_layer(L) for L in layers]
        out = eng.forward_stack(ids, x, path)
    finally:
        eng.close()
    ref, clear = oracle_stack(oracle_mod, layers, x)
    check_stack(oracle_mod, f"stack q8 shared path {path}", ref, out, clear)
