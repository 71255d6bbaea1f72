"""The GGUF header reader (include/gyro_gguf.h), on the CPU: the cases of src/gguf.zig's own
tests (expert slices of the real model's down tensor, truncation at every byte, overlapping
ranges and overflow, duplicate keys and invalid booleans, unknown tensor types), plus metadata,
alignment, a written file whose expert slices round-trip through gg_open, and the rotation
metadata check of src/gguf.zig:182-250."""
import numpy as np
import pytest

from gguf_fixture import GgufBuilder
from gyrodx import gguf


def kind(fn):
    with pytest.raises(gguf.GgufError) as e:
        fn()
    return e.value.kind


def test_expert_slices_use_block_bytes_and_absolute_offsets():
    """The real model's down tensor: 640 x 2560 TQ2_T weights per expert, 256 experts."""
    f = GgufBuilder().header(1, 0).tensor("blk.0.ffn_down_exps.weight", (640, 2560, 256), 144, 0).pad()
    payload = 435200 * 256
    m = gguf.parse(f.bytes(), len(f.bytes()) + payload)
    off, n = m.expert_range("blk.0.ffn_down_exps.weight", 255)
    assert n == 435200 == 640 // 128 * 34 * 2560
    assert off == m.data_offset + 435200 * 255
    assert kind(lambda: m.expert_range("blk.0.ffn_down_exps.weight", 256)) == "InvalidExpert"
    full = len(f.bytes()) + payload
    for end in range(len(f.bytes())):
        assert kind(lambda: gguf.parse(f.bytes()[:end], full)) == "UnexpectedEnd", end


def test_overlapping_ranges_and_overflow():
    f = GgufBuilder().header(2, 0).tensor("a", (32,), 0, 0).tensor("b", (32,), 0, 32).pad()
    assert kind(lambda: gguf.parse(f.bytes(), 4096)) == "OverlappingTensors"
    f = GgufBuilder().header(1, 0).tensor("a", (2 ** 64 - 1, 2), 0, 0).pad()
    assert kind(lambda: gguf.parse(f.bytes(), 2 ** 64 - 1)) == "IntegerOverflow"


def test_duplicate_keys_and_invalid_booleans():
    f = GgufBuilder().header(0, 2)
    for _ in range(2):
        f.str("a").u32(4).u32(1)
    assert kind(lambda: gguf.parse(f.pad().bytes(), 4096)) == "DuplicateKey"
    f = GgufBuilder().header(0, 1).str("a").u32(7).u8(2).pad()
    assert kind(lambda: gguf.parse(f.bytes(), 4096)) == "InvalidBoolean"


def test_unknown_tensor_type_keeps_no_size():
    f = GgufBuilder().header(1, 0).tensor("unknown", (128, 2, 4), 999, 0).pad()
    m = gguf.parse(f.bytes(), 4096)
    assert m.tensors()[0].byte_length is None
    assert kind(lambda: m.expert_range("unknown", 0)) == "UnsupportedTensorType"


def test_header_checks_and_metadata():
    assert kind(lambda: gguf.parse(GgufBuilder().header(0, 0, magic=b"GGUX").pad().bytes(), 64)) == "BadMagic"
    assert kind(lambda: gguf.parse(GgufBuilder().header(0, 0, version=2).pad().bytes(), 64)) == "UnsupportedVersion"
    f = GgufBuilder().header(1, 2).kv_u32("general.alignment", 64).kv_str("general.name", "x")
    f.tensor("t", (128, 3), 145, 64).pad(64)
    m = gguf.parse(f.bytes(), len(f.bytes()) + 64 + 26 * 3)
    assert m.alignment == 64 and m.data_offset % 64 == 0 and m.metadata_u64("general.alignment") == 64
    assert m.tensor("t").byte_length == 26 * 3 and m.tensor("t").file_offset == m.data_offset + 64
    assert kind(lambda: m.metadata_u64("general.name")) == "InvalidMetadata"
    f = GgufBuilder().header(1, 1).kv_u32("general.alignment", 48).tensor("t", (4,), 0, 0).pad()
    assert kind(lambda: gguf.parse(f.bytes(), 4096)) == "InvalidAlignment"
    f = GgufBuilder().header(1, 0).tensor("t", (4,), 0, 16).pad()
    assert kind(lambda: gguf.parse(f.bytes(), 4096)) == "InvalidAlignment"
    assert gguf.is_expert_tensor("blk.3.ffn_up_exps.weight") and not gguf.is_expert_tensor("blk.3.ffn_up.weight")


def test_written_file_expert_slices(tmp_path):
    """A file with three TQ2_T expert tensors: every expert's slice read back through gg_open and
    the mapped loader equals the bytes written."""
    rng = np.random.default_rng(5)
    E, F, NE = 256, 128, 3
    mats = {"gate": rng.integers(0, 256, (NE, F, E // 128 * 34), dtype=np.uint8),
            "up": rng.integers(0, 256, (NE, F, E // 128 * 34), dtype=np.uint8),
            "down": rng.integers(0, 256, (NE, E, F // 128 * 34), dtype=np.uint8)}
    f = GgufBuilder().header(3, 0)
    off = 0
    offs = {}
    for p, dims in (("gate", (E, F, NE)), ("up", (E, F, NE)), ("down", (F, E, NE))):
        offs[p] = off
        f.tensor(f"blk.0.ffn_{p}_exps.weight", dims, 144, off)
        off += (mats[p].nbytes + 31) // 32 * 32
    f.pad()
    data = bytearray(off)
    for p in mats:
        data[offs[p]:offs[p] + mats[p].nbytes] = mats[p].tobytes()
    path = tmp_path / "experts.gguf"
    path.write_bytes(f.bytes() + bytes(data))
    got = gguf.load_layer_experts(str(path), 0)
    assert (got["E"], got["F"], got["n_expert"]) == (E, F, NE)
    for p in mats:
        for e in range(NE):
            np.testing.assert_array_equal(got[p][e], mats[p][e])


def gyro_meta(f, names, widths, signs, **over):
    kv = {"agention.trellis.state_bits": ("u32", 15), "prism.hadamard.version": ("u32", 1),
          "prism.hadamard.block_size": ("u32", 128),
          "prism.hadamard.transform": ("str", "normalized-sylvester-walsh-hadamard"),
          "prism.hadamard.axis": ("str", "input-last-dimension"), "prism.hadamard.sign_mode": ("str", "explicit"),
          "prism.hadamard.weight_names": ("strs", names), "prism.hadamard.sign_widths": ("i32s", widths),
          "prism.hadamard.sign_values": ("i32s", signs)}
    kv.update(over)
    kv = {k: v for k, v in kv.items() if v is not None}
    return kv


def gyro_file(**over):
    kv = gyro_meta(None, ["w"], [128], [1, -1] * 64, **over)
    f = GgufBuilder().header(1, len(kv))
    for k, (kind, v) in kv.items():
        {"u32": f.kv_u32, "str": f.kv_str, "strs": f.kv_strs, "i32s": f.kv_i32s, "bool": f.kv_bool}[kind](k, v)
    f.tensor("w", (128, 4), 144, 0).pad()
    return gguf.parse(f.bytes(), len(f.bytes()) + 4 * 34)


def test_validate_gyro_metadata():
    """src/gguf.zig:182-250: the released version-1 rotation metadata is accepted; each departure
    is refused with the reference's error kind."""
    gyro_file().validate_gyro()
    assert kind(lambda: gyro_file(**{"agention.trellis.state_bits": ("u32", 16)}).validate_gyro()) == "UnsupportedGyroMetadata"
    assert kind(lambda: gyro_file(**{"prism.hadamard.block_size": ("u32", 96)}).validate_gyro()) == "InvalidMetadata"
    assert kind(lambda: gyro_file(**{"prism.hadamard.axis": ("str", "output")}).validate_gyro()) == "UnsupportedGyroMetadata"
    assert kind(lambda: gyro_file(**{"prism.hadamard.sign_values": ("i32s", [1, 0] * 64)}).validate_gyro()) == "InvalidMetadata"
    assert kind(lambda: gyro_file(**{"prism.hadamard.sign_values": ("i32s", [1] * 127)}).validate_gyro()) == "InvalidMetadata"
    assert kind(lambda: gyro_file(**{"prism.hadamard.weight_names": ("strs", ["w", "w"])}).validate_gyro()) == "InvalidMetadata"
    assert kind(lambda: gyro_file(**{"prism.hadamard.weight_names": ("strs", ["missing"])}).validate_gyro()) == "InvalidMetadata"
    assert kind(lambda: gyro_file(**{"prism.hadamard.sign_widths": ("i32s", [256]),
                                     "prism.hadamard.sign_values": ("i32s", [1] * 256)}).validate_gyro()) == "InvalidMetadata"
    assert kind(lambda: gyro_file(**{"prism.hadamard.sign_mode": ("str", "identity")}).validate_gyro()) == "InvalidMetadata"
    gyro_file(**{"prism.hadamard.sign_mode": ("str", "identity"), "prism.hadamard.sign_widths": None,
                 "prism.hadamard.sign_values": None}).validate_gyro()
    assert kind(lambda: gyro_file(**{"prism.hadamard.tied_output": ("bool", True)}).validate_gyro()) == "UnsupportedGyroMetadata"
    assert kind(lambda: gyro_file(**{"prism.hadamard.transform": None}).validate_gyro()) == "InvalidMetadata"


def test_metadata_values():
    m = gyro_file()
    assert m.metadata("prism.hadamard.weight_names") == ["w"]
    assert m.metadata("prism.hadamard.sign_values")[:4] == [1, -1, 1, -1]
    assert m.metadata("prism.hadamard.axis") == "input-last-dimension"
    assert m.has("prism.hadamard.version") and not m.has("nope")


def small_layer(**kw):
    from gyrodx import synth
    return synth.make_layer(31, E=512, F=256, n_expert=4, n_used=2, **kw)


def test_load_layer_refuses_what_the_model_loader_refuses(tmp_path):
    """src/model.zig:312 (block size 128), :421-429 (only expert projections are listed) and
    src/gpu_engine.zig:404 (up-projection signs must be the gate's)."""
    from gguf_fixture import write_layer_file
    L = small_layer()
    names = [f"blk.0.ffn_{p}_exps.weight" for p in ("gate", "up", "down")]
    cases = {"block256": dict(block_size=256), "up_only": dict(listed=[names[1], names[2]]),
             "router_listed": dict(listed=names + ["blk.0.ffn_gate_inp.weight"])}
    for what, kw in cases.items():
        path = tmp_path / f"{what}.gguf"
        write_layer_file(path, L, **kw)
        gguf.open_model(str(path)).validate_gyro()  # the rotation metadata itself is valid
        with pytest.raises(gguf.UnsupportedConfiguration):
            gguf.load_layer(str(path), 0)
    # The released layout loads, with the gate's signs shared by up.
    path = tmp_path / "ok.gguf"
    write_layer_file(path, L)
    G = gguf.load_layer(str(path), 0)
    np.testing.assert_array_equal(G.gate_signs, L.gate_signs)
    np.testing.assert_array_equal(G.down_signs, L.down_signs)
    assert G.SF == 0


@pytest.mark.parametrize("sh_type", [8, 30, 0])
def test_load_layer_reads_the_shared_expert(tmp_path, sh_type):
    """blk.<l>.ffn_{gate,up,down}_shexp.weight and ffn_gate_inp_shexp.weight (src/model.zig:413-416)
    round-trip in Q8_0, bf16 and fp32."""
    from gguf_fixture import write_layer_file
    L = small_layer(SF=64, sh_type=sh_type)
    path = tmp_path / "shared.gguf"
    write_layer_file(path, L)
    G = gguf.load_layer(str(path), 0)
    assert (G.SF, G.sh_type) == (64, sh_type)
    for name in ("sh_gate", "sh_up", "sh_down"):
        np.testing.assert_array_equal(G.__dict__[name].view(np.uint8).ravel(),
                                      np.ascontiguousarray(getattr(L, name)).view(np.uint8).ravel())
    np.testing.assert_array_equal(G.sh_gate_inp, L.sh_gate_inp)


def test_validate_gyro_compares_widths_as_u64():
    """src/gguf.zig:237 compares a listed tensor's first dimension with the sign widths as u64:
    a dimension of 2^32 + 128 (kept with an unknown tensor type, so no byte range) is not width
    128. A Gyro tensor in the file makes the rotation metadata apply."""
    def build(dim0):
        kv = gyro_meta(None, ["w"], [128], [1, -1] * 64)
        f = GgufBuilder().header(2, len(kv))
        for k, (kd, v) in kv.items():
            {"u32": f.kv_u32, "str": f.kv_str, "strs": f.kv_strs, "i32s": f.kv_i32s, "bool": f.kv_bool}[kd](k, v)
        f.tensor("g", (128, 4), 144, 0).tensor("w", (dim0, 1), 999, 160).pad()
        return gguf.parse(f.bytes(), len(f.bytes()) + 4 * 34 + 64)
    build(128).validate_gyro()
    assert kind(lambda: build(2 ** 32 + 128).validate_gyro()) == "InvalidMetadata"
