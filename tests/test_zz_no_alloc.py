"""The no-allocation decode entry point (gm_forward_decode_noalloc) against gm_forward on the
decode path, through the C ABI: outputs equal bit for bit on two calls in a row, the second
with fewer tokens, on a uniform TQ2_T layer (moe_decode_gu / moe_decode_down) and on a mixed-type
layer with a shared expert (moe_decode_gu_x / moe_decode_down_x, the shared rows in the scratch
array) and at hidden 2560 / F 640 / top-10 with a Q8_0 shared expert (mv_q8 and ew ahead of the
routed kernels, every intermediate in the scratch array). Inputs and outputs are torch device tensors; the first call is queued on the engine's
compute stream, the second on a torch stream.
"""
import numpy as np
import pytest
import torch

from gyrodx import synth
from gyrodx.engine import PATH_DECODE, Engine

pytestmark = pytest.mark.gpu


def _layer(kind):
    if kind == "tq2":
        return synth.make_layer(7, E=2048, F=512, n_expert=256, n_used=8)
    if kind == "coder_q8_shared":  # the shared expert in the mv kernels, its buffers in the scratch array
        return synth.make_layer(9, E=2560, F=640, n_expert=64, n_used=10, SF=640, sh_type=8)
    return synth.make_layer(8, E=2048, F=512, n_expert=64, n_used=8, mixed_types=True, SF=512)


@pytest.mark.parametrize("kind", ["tq2", "mixed_shared", "coder_q8_shared"])
def test_noalloc_matches_forward(kind):
    layer = _layer(kind)
    eng = Engine(max_tok=8)
    try:
        li = eng.add_layer(layer)
        side = torch.cuda.Stream()
        for call, n in enumerate((8, 3)):
            print(f"noalloc {kind}: call {call}, {n} tokens", flush=True)
            x = synth.make_tokens(300 + call, n, layer.E)
            ref = eng.forward(li, x, PATH_DECODE)
            ref_ids, _ = eng.last_routes(n)
            xd = torch.from_numpy(x).to("cuda")
            od = torch.full((n, layer.E), float("nan"), device="cuda")
            torch.cuda.synchronize()
            if call == 0:
                eng.forward_decode_noalloc(li, xd.data_ptr(), n, od.data_ptr(), 0)
            else:
                with torch.cuda.stream(side):
                    eng.forward_decode_noalloc(li, xd.data_ptr(), n, od.data_ptr(), side.cuda_stream)
            torch.cuda.synchronize()
            out = od.cpu().numpy()
            assert np.isfinite(out).all()
            diff = np.flatnonzero(out.view(np.uint32) != ref.view(np.uint32))
            assert diff.size == 0, f"{diff.size} values differ from gm_forward (first {diff[:4]})"
            ids, _ = eng.last_routes(n)  # the engine's own buffers still hold gm_forward's routes
            assert (ids == ref_ids).all()
    finally:
        eng.close()


def test_noalloc_refuses_more_than_eight_tokens():
    layer = _layer("tq2")
    eng = Engine(max_tok=16)
    try:
        li = eng.add_layer(layer)
        xd = torch.zeros((9, layer.E), device="cuda")
        od = torch.zeros((9, layer.E), device="cuda")
        with pytest.raises(RuntimeError, match="1 to 8 tokens"):
            eng.forward_decode_noalloc(li, xd.data_ptr(), 9, od.data_ptr(), 0)
        with pytest.raises(RuntimeError):
            eng.forward_decode_noalloc(li, xd.data_ptr(), 0, od.data_ptr(), 0)
    finally:
        eng.close()
