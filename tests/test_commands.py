"""The conformance commands' host side (gyrodx.commands) on the CPU: its strict decoder equals
the oracle's bit for bit on the validateGyro recipe of src/native.zig:119-152 (all eight types,
the twelve edge scales: zeros, subnormals, the normal boundary, one, the largest finite) and on
random blocks; the recipe's LCG state runs on across types; the expert bundle of a written
file is the gate, up and down slices of src/plan.zig:17-31, and other architectures, missing
layers and incomplete sets are refused."""
import numpy as np
import pytest

from gguf_fixture import write_layer_file
from gyrodx import CODEBOOK, commands, gguf, synth


def test_decoder_matches_oracle_on_recipe_and_random_blocks(oracle_mod):
    book = CODEBOOK.read_bytes()
    state = 0x4759524F
    rng = np.random.default_rng(1)
    for type_id, (_, _, bb) in commands.TYPES.items():
        enc, state2 = commands.recipe_blocks(type_id, state)
        assert state2 != state
        state = state2
        rnd = rng.integers(0, 256, bb * 40, dtype=np.uint8)
        rnd.reshape(40, bb)[:, 1] &= 0x7B  # finite scales
        for blocks in (enc, rnd):
            rc, want = oracle_mod.decode_row(type_id, blocks, blocks.size // bb * 128)
            assert rc == 0
            got = commands.decode_row(type_id, blocks, book)
            np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_expert_bundle(tmp_path):
    layer = synth.make_layer(3, E=256, F=256, n_expert=4, n_used=2)
    path = tmp_path / "m.gguf"
    write_layer_file(path, layer, arch="qwen4exp")
    m = gguf.open_model(str(path))
    try:
        b = commands.expert_bundle(m, 0, 3)
        assert b == [m.expert_range(f"blk.0.ffn_{k}_exps.weight", 3) for k in ("gate", "up", "down")]
        with pytest.raises(commands.CommandError, match="InvalidExpert"):
            commands.expert_bundle(m, 1, 0)
        with pytest.raises(gguf.GgufError):
            commands.expert_bundle(m, 0, 4)
    finally:
        m.close()
    write_layer_file(tmp_path / "o.gguf", layer, arch="other")
    m = gguf.open_model(str(tmp_path / "o.gguf"))
    try:
        with pytest.raises(commands.CommandError, match="UnsupportedArchitecture"):
            commands.expert_bundle(m, 0, 0)
    finally:
        m.close()


def test_usage():
    assert commands.main([]) == 2 and commands.main(["gyro"]) == 2


def test_type_names_follow_the_type_table():
    """validateGyro prints info.name of the type table (src/gyro.zig:33-40): id, name, k, steps,
    block bytes."""
    from gyrodx import synth
    from gyrodx.commands import TYPE_NAMES
    table = {144: ("TQ2_T", 8, 32, 34), 145: ("TQK6", 6, 32, 26), 146: ("TQK7", 7, 32, 30),
             147: ("TQP5", 5, 64, 42), 148: ("TQP6", 6, 64, 50), 149: ("TQP7", 7, 64, 58),
             150: ("TQK5", 5, 32, 22), 151: ("TQK4", 4, 32, 18)}
    assert TYPE_NAMES == {i: v[0] for i, v in table.items()}
    assert synth.TYPES == {i: v[1:] for i, v in table.items()}
