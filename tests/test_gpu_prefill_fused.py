"""The persistent prefill GEMM launch (moe_prefill_gemm: the gate/up and down units of
src/engine.zig:567-633 from one work queue) against the two-launch path (moe_prefill_gu,
moe_prefill_down) and the CPU oracle.

Both paths run the same units on the same tiles, so their outputs must be equal bit for bit; the
persistent one must also meet the oracle bar of the prefill tests (relative RMS 2e-3, cosine
0.9999 against the fp32 results of src/engine.zig:520-653). Shapes: the 1024-token Zipf layer of
the benchmark, the real model's expert shape (hidden 2560, F 640 with its odd block count per
down row, top-10), the widest hidden (4096, sixteen down units per tile) with top-16, F 384 with
top-6, and batches of 1 and 33 tokens (one and a few tiles). The forced give-up (a spin limit of
zero polls) must leave gm_forward's result unchanged: the call is recomputed with two launches.

moe_prefill_gemm_x is the same queue over the type-generic units (moe_prefill_gu_x,
moe_prefill_down_x) for layers whose experts and projections mix Gyro types or use one type other
than TQ2_T: against its two launches bit for bit and against the oracle, on the mixed-quant layer
with its bf16 shared expert, the real model's expert shape in GGUF 148 with a Zipf router, and a
mixed layer at F 384 / top-6; its forced give-up is recomputed as above.

moe_prefill_gemm_s is the same launch with small-tile units for sort tiles of at most 16 rows (8
past hidden 2048); the engine takes it when the average expert segment is short (tokens x top-k
at most 8 x experts) and the shape has them (hidden and F multiples of 512, hidden at most 4096).
Forced on for every call, it must give the bits of moe_prefill_gemm and of the two launches, on
shapes where tiles of 1 to 16 rows are common and where the large tiles of a Zipf router mix in.
"""
import os

import numpy as np
import pytest

from gyrodx import synth
from gyrodx.engine import PATH_PREFILL, Engine

pytestmark = pytest.mark.gpu
REL_RMS, COSINE = 2e-3, 0.9999


def make_engine(max_tok, fused, spin_limit=None, small=None):
    """small: GYRO_PREFILL_SMALL ('0' never moe_prefill_gemm_s, '2' always where the shape has
    small units, None the engine's own choice)."""
    saved = {k: os.environ.get(k) for k in ("GYRO_PREFILL_FUSED", "GYRO_PREFILL_SPIN_LIMIT", "GYRO_PREFILL_SMALL")}
    os.environ["GYRO_PREFILL_FUSED"] = "1" if fused else "0"
    if small is not None:
        os.environ["GYRO_PREFILL_SMALL"] = small
    if spin_limit is not None:
        os.environ["GYRO_PREFILL_SPIN_LIMIT"] = str(spin_limit)
    try:
        return Engine(max_tok=max_tok)
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


SHAPES = [
    # E, F, experts, top-k, tokens, extra make_layer arguments
    (2048, 512, 256, 8, 1024, {"zipf": 1.1}),
    (2560, 640, 64, 10, 300, {}),
    (4096, 256, 16, 16, 64, {}),
    (2048, 384, 64, 6, 200, {"signs": False}),
    (1024, 256, 32, 4, 1, {}),
    (1024, 256, 32, 4, 33, {"zipf": 1.1}),
]


@pytest.mark.parametrize("E,F,NE,U,n,kw", SHAPES,
                         ids=[f"E{s[0]}-F{s[1]}-x{s[2]}-top{s[3]}-n{s[4]}" + "".join(f"-{k}" for k in s[5]) for s in SHAPES])
def test_persistent_gemm_matches_two_launches(oracle_mod, E, F, NE, U, n, kw):
    L = synth.make_layer(1500 + E // 128 + F // 64 + U, E=E, F=F, n_expert=NE, n_used=U, **kw)
    x = synth.make_tokens(1501 + n, n, E, bf16=True)
    outs = {}
    for fused in (True, False):
        eng = make_engine(max(n, 64), fused)
        try:
            eng.add_layer(L)
            print(f"prefill E={E} F={F} experts={NE} top-{U} n={n} {'persistent' if fused else 'two launches'}",
                  flush=True)
            outs[fused] = eng.forward(0, x, PATH_PREFILL)
            if fused:
                tiles = eng.last_tiles()
                print(f"  {len(tiles)} tiles", flush=True)
        finally:
            eng.close()
    np.testing.assert_array_equal(outs[True].view(np.uint32), outs[False].view(np.uint32))
    ref = oracle_mod.OracleLayer(L).forward(x)
    r, c = oracle_mod.rel_rms(ref, outs[True]), oracle_mod.cosine(ref, outs[True])
    print(f"  bit-equal to the two-launch path; rel_rms {r:.3e} cosine {c:.8f}", flush=True)
    assert r <= REL_RMS and c >= COSINE




def test_persistent_gemm_give_up_recomputes():
    """With a spin limit of zero polls a down unit whose tile is not finished gives up at once.
    The give-up word is sticky: the sort of a later call or layer does not clear it, only the host
    does after reading it. So gm_forward and gm_forward_stack (two layers) recompute with two
    launches and return the two-launch engine's outputs bit for bit, and gm_run over two calls
    either reports the give-up or returns those outputs bit for bit."""
    n = 1024
    L = synth.make_layer(1560, zipf=1.1)
    S = synth.make_stack(1562, 2, zipf=1.1)
    x = synth.make_tokens(1561, 2 * n, bf16=True)
    ref_eng = make_engine(n, False)
    try:
        ref_eng.add_layer(L)
        sids = [ref_eng.add_layer(s) for s in S]
        ref = ref_eng.forward(0, x[:n], PATH_PREFILL)
        ref_stack = ref_eng.forward_stack(sids, x[:n], PATH_PREFILL)
        ref_eng.set_tokens(x)
        ref_eng.run(PATH_PREFILL, n, 2, [0])
        ref_run = ref_eng.read_outputs(2 * n)
    finally:
        ref_eng.close()
    eng = make_engine(n, True, spin_limit=0)
    try:
        eng.add_layer(L)
        sids = [eng.add_layer(s) for s in S]
        print("persistent prefill GEMM, spin limit 0: gm_forward", flush=True)
        out = eng.forward(0, x[:n], PATH_PREFILL)
        np.testing.assert_array_equal(out.view(np.uint32), ref.view(np.uint32))
        print("  gm_forward_stack over 2 layers", flush=True)
        out = eng.forward_stack(sids, x[:n], PATH_PREFILL)
        np.testing.assert_array_equal(out.view(np.uint32), ref_stack.view(np.uint32))
        eng.set_tokens(x)
        try:
            eng.run(PATH_PREFILL, n, 2, [0])
            got = eng.read_outputs(2 * n)
            np.testing.assert_array_equal(got.view(np.uint32), ref_run.view(np.uint32))
            print("  gm_run: no unit gave up; outputs equal the two-launch run", flush=True)
        except RuntimeError as err:
            assert "gave up waiting" in str(err), err
            print("  gm_run reported the give-up", flush=True)
    finally:
        eng.close()


SMALL_SHAPES = [
    # E, F, experts, top-k, tokens, extra make_layer arguments
    (2048, 512, 256, 8, 128, {}),
    (2048, 512, 256, 8, 256, {"zipf": 1.1}),
    (1024, 512, 64, 4, 37, {}),
    (4096, 512, 64, 8, 100, {}),
    (3072, 1024, 32, 6, 1, {"signs": False}),
]


@pytest.mark.parametrize("E,F,NE,U,n,kw", SMALL_SHAPES,
                         ids=[f"E{s[0]}-F{s[1]}-x{s[2]}-top{s[3]}-n{s[4]}" + "".join(f"-{k}" for k in s[5]) for s in SMALL_SHAPES])
def test_small_units_match(oracle_mod, E, F, NE, U, n, kw):
    L = synth.make_layer(1600 + E // 128 + F // 64 + U, E=E, F=F, n_expert=NE, n_used=U, **kw)
    x = synth.make_tokens(1601 + n, n, E, bf16=True)
    outs = {}
    for name, fused, small in (("moe_prefill_gemm_s", True, "2"), ("moe_prefill_gemm", True, "0"),
                               ("two launches", False, "0")):
        eng = make_engine(max(n, 64), fused, small=small)
        try:
            eng.add_layer(L)
            print(f"prefill E={E} F={F} experts={NE} top-{U} n={n} {name}", flush=True)
            outs[name] = eng.forward(0, x, PATH_PREFILL)
            if name == "moe_prefill_gemm_s":
                rows = [t[2] for t in eng.last_tiles()]
                print(f"  {len(rows)} tiles, {sum(r <= (16 if E <= 2048 else 8) for r in rows)} small", flush=True)
        finally:
            eng.close()
    for name in ("moe_prefill_gemm", "two launches"):
        np.testing.assert_array_equal(outs["moe_prefill_gemm_s"].view(np.uint32), outs[name].view(np.uint32),
                                      err_msg=name)
    ref = oracle_mod.OracleLayer(L).forward(x)
    r, c = oracle_mod.rel_rms(ref, outs["moe_prefill_gemm_s"]), oracle_mod.cosine(ref, outs["moe_prefill_gemm_s"])
    print(f"  bit-equal; rel_rms {r:.3e} cosine {c:.8f}", flush=True)
    assert r <= REL_RMS and c >= COSINE


X_SHAPES = [
    # E, F, experts, top-k, tokens, extra make_layer arguments
    (2048, 512, 256, 8, 512, {"mixed_types": True, "SF": 1024}),
    (2560, 640, 64, 10, 300, {"type_id": 148, "zipf": 1.1}),
    (1024, 384, 32, 6, 100, {"mixed_types": True, "signs": False}),
    (1024, 256, 32, 4, 1, {"type_id": 151}),
]


@pytest.mark.parametrize("E,F,NE,U,n,kw", X_SHAPES,
                         ids=[f"E{s[0]}-F{s[1]}-x{s[2]}-top{s[3]}-n{s[4]}" + "".join(f"-{k}{v}" for k, v in s[5].items())
                              for s in X_SHAPES])
def test_persistent_gemm_x_matches_two_launches(oracle_mod, E, F, NE, U, n, kw):
    L = synth.make_layer(1700 + E // 128 + F // 64 + U, E=E, F=F, n_expert=NE, n_used=U, **kw)
    x = synth.make_tokens(1701 + n, n, E, bf16=True)
    outs = {}
    for fused in (True, False):
        eng = make_engine(max(n, 64), fused)
        try:
            eng.add_layer(L)
            print(f"prefill E={E} F={F} experts={NE} top-{U} n={n} {kw} "
                  f"{'moe_prefill_gemm_x' if fused else 'moe_prefill_gu_x + moe_prefill_down_x'}", flush=True)
            outs[fused] = eng.forward(0, x, PATH_PREFILL)
        finally:
            eng.close()
    np.testing.assert_array_equal(outs[True].view(np.uint32), outs[False].view(np.uint32))
    ref = oracle_mod.OracleLayer(L).forward(x)
    r, c = oracle_mod.rel_rms(ref, outs[True]), oracle_mod.cosine(ref, outs[True])
    print(f"  bit-equal to the two-launch path; rel_rms {r:.3e} cosine {c:.8f}", flush=True)
    assert r <= REL_RMS and c >= COSINE


def test_persistent_gemm_x_give_up_recomputes():
    """moe_prefill_gemm_x with a spin limit of zero polls: gm_forward recomputes with the two
    type-generic launches and returns their outputs bit for bit; gm_run over two calls either
    reports the give-up or returns the two-launch run's outputs bit for bit."""
    n = 512
    L = synth.make_layer(1760, mixed_types=True, zipf=1.1)
    x = synth.make_tokens(1761, 2 * n, bf16=True)
    ref_eng = make_engine(n, False)
    try:
        ref_eng.add_layer(L)
        ref = ref_eng.forward(0, x[:n], PATH_PREFILL)
        ref_eng.set_tokens(x)
        ref_eng.run(PATH_PREFILL, n, 2, [0])
        ref_run = ref_eng.read_outputs(2 * n)
    finally:
        ref_eng.close()
    eng = make_engine(n, True, spin_limit=0)
    try:
        eng.add_layer(L)
        print("moe_prefill_gemm_x, spin limit 0: gm_forward", flush=True)
        out = eng.forward(0, x[:n], PATH_PREFILL)
        np.testing.assert_array_equal(out.view(np.uint32), ref.view(np.uint32))
        eng.set_tokens(x)
        try:
            eng.run(PATH_PREFILL, n, 2, [0])
            got = eng.read_outputs(2 * n)
            np.testing.assert_array_equal(got.view(np.uint32), ref_run.view(np.uint32))
            print("  gm_run: no unit gave up; outputs equal the two-launch run", flush=True)
        except RuntimeError as err:
            assert "gave up waiting" in str(err), err
            print("  gm_run reported the give-up", flush=True)
    finally:
        eng.close()
