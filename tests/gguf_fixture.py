"""Byte builder for GGUF v3 test files: header, metadata entries, tensor infos, padding to the
alignment, tensor data (the file layout src/gguf.zig:263-330 parses)."""
import struct


class GgufBuilder:
    def __init__(self):
        self.b = bytearray()

    def u8(self, v):
        self.b += struct.pack("<B", v)
        return self

    def u32(self, v):
        self.b += struct.pack("<I", v)
        return self

    def u64(self, v):
        self.b += struct.pack("<Q", v)
        return self

    def str(self, s):
        s = s.encode() if isinstance(s, str) else s
        self.u64(len(s))
        self.b += s
        return self

    def header(self, n_tensors, n_kv, version=3, magic=b"GGUF"):
        self.b += magic
        return self.u32(version).u64(n_tensors).u64(n_kv)

    def kv_u32(self, key, v):
        return self.str(key).u32(4).u32(v)

    def kv_str(self, key, v):
        return self.str(key).u32(8).str(v)

    def kv_f32(self, key, v):
        self.str(key).u32(6)
        self.b += struct.pack("<f", v)
        return self

    def kv_bool(self, key, v):
        return self.str(key).u32(7).u8(1 if v else 0)

    def kv_i32s(self, key, vals):
        self.str(key).u32(9).u32(5).u64(len(vals))
        for v in vals:
            self.b += struct.pack("<i", int(v))
        return self

    def kv_strs(self, key, vals):
        self.str(key).u32(9).u32(8).u64(len(vals))
        for v in vals:
            self.str(v)
        return self

    def tensor(self, name, dims, type_id, offset):
        self.str(name).u32(len(dims))
        for d in dims:
            self.u64(d)
        return self.u32(type_id).u64(offset)

    def pad(self, alignment=32):
        while len(self.b) % alignment:
            self.b += b"\0"
        return self

    def bytes(self):
        return bytes(self.b)


def write_layer_file(path, L, arch="gyrotest", block_size=128, listed=None):
    """One MoE layer as a GGUF file: blk.0.ffn_gate_inp.weight (fp32 router, dims (E, n_expert)),
    blk.0.ffn_{gate,up,down}_exps.weight (Gyro experts), the expert counts and scale under
    `arch`, and the released rotation metadata with explicit signs for widths E (gate, up) and
    F (down), listing `listed` (default: the three expert tensors). With a shared expert (L.SF)
    also blk.0.ffn_{gate,up,down}_shexp.weight in L.sh_type (dims (E, SF), (E, SF), (SF, E))
    and the fp32 blk.0.ffn_gate_inp_shexp.weight (dims (E,))."""
    import numpy as np
    ty = int(L.types[0, 0])
    names = [f"blk.0.ffn_{p}_exps.weight" for p in ("gate", "up", "down")]
    listed = names if listed is None else listed
    kv = [("general.alignment", "u32", 32), ("general.architecture", "str", arch),
          (f"{arch}.expert_count", "u32", L.n_expert), (f"{arch}.expert_used_count", "u32", L.n_used),
          (f"{arch}.block_count", "u32", 1),
          ("agention.trellis.state_bits", "u32", 15), ("prism.hadamard.version", "u32", 1),
          ("prism.hadamard.block_size", "u32", block_size),
          ("prism.hadamard.transform", "str", "normalized-sylvester-walsh-hadamard"),
          ("prism.hadamard.axis", "str", "input-last-dimension"), ("prism.hadamard.sign_mode", "str", "explicit"),
          ("prism.hadamard.weight_names", "strs", list(listed)),
          ("prism.hadamard.sign_widths", "i32s", [L.E, L.F]),
          ("prism.hadamard.sign_values", "i32s", list(L.gate_signs.astype(int)) + list(L.down_signs.astype(int)))]
    if L.expert_weights_scale:
        kv.append((f"{arch}.expert_weights_scale", "f32", L.expert_weights_scale))
    blobs = [("blk.0.ffn_gate_inp.weight", (L.E, L.n_expert), 0, np.ascontiguousarray(L.router, np.float32)),
             (names[0], (L.E, L.F, L.n_expert), ty, np.stack(L.gate)),
             (names[1], (L.E, L.F, L.n_expert), ty, np.stack(L.up)),
             (names[2], (L.F, L.E, L.n_expert), ty, np.stack(L.down))]
    if L.SF:
        blobs += [("blk.0.ffn_gate_shexp.weight", (L.E, L.SF), L.sh_type, np.ascontiguousarray(L.sh_gate)),
                  ("blk.0.ffn_up_shexp.weight", (L.E, L.SF), L.sh_type, np.ascontiguousarray(L.sh_up)),
                  ("blk.0.ffn_down_shexp.weight", (L.SF, L.E), L.sh_type, np.ascontiguousarray(L.sh_down)),
                  ("blk.0.ffn_gate_inp_shexp.weight", (L.E,), 0, np.ascontiguousarray(L.sh_gate_inp, np.float32))]
    f = GgufBuilder().header(len(blobs), len(kv))
    for key, kind, v in kv:
        {"u32": f.kv_u32, "str": f.kv_str, "strs": f.kv_strs, "i32s": f.kv_i32s, "f32": f.kv_f32}[kind](key, v)
    off, offs = 0, []
    for name, dims, t, arr in blobs:
        f.tensor(name, dims, t, off)
        offs.append(off)
        off += (arr.nbytes + 31) // 32 * 32
    f.pad()
    data = bytearray(off)
    for (_, _, _, arr), o in zip(blobs, offs):
        data[o:o + arr.nbytes] = arr.tobytes()
    with open(path, "wb") as fh:
        fh.write(f.bytes())
        fh.write(bytes(data))
