"""ctypes binding of the GGUF reader (include/gyro_gguf.h) and the routed-expert loader above it.

`open_model(path)` parses a GGUF v3 header as src/gguf.zig:263-330 does; `expert_range` slices a
rank-3 expert tensor (src/gguf.zig:138-143). `load_layer_experts` maps a file and returns, for
each expert, its gate, up and down matrices as views of the file in the engine's layout
([rows][blocks x block bytes]), which is exactly the GGUF expert slice: a gate or up tensor
"blk.<l>.ffn_{gate,up}_exps.weight" has dims (E, F, n_expert), a down tensor (F, E, n_expert).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import engine as _engine

GYRO_BLOCK_BYTES = {144: 34, 145: 26, 146: 30, 147: 42, 148: 50, 149: 58, 150: 22, 151: 18}


class GgufError(RuntimeError):
    NAMES = {-1: "UnexpectedEnd", -2: "BadMagic", -3: "UnsupportedVersion", -4: "InvalidType",
             -5: "InvalidBoolean", -6: "LimitExceeded", -7: "IntegerOverflow", -8: "InvalidAlignment",
             -9: "InvalidDimensions", -10: "DuplicateKey", -11: "DuplicateTensor", -12: "InvalidTensorRange",
             -13: "OverlappingTensors", -14: "UnsupportedTensorType", -15: "InvalidExpert",
             -16: "InvalidMetadata", -17: "IO", -18: "NotFound", -19: "UnsupportedGyroMetadata",
             -20: "OutOfMemory"}

    def __init__(self, code: int, what: str):
        self.code = code
        self.kind = self.NAMES.get(code, str(code))
        super().__init__(f"{what}: {self.kind}")


class UnsupportedConfiguration(GgufError):
    """A well-formed file the model loader refuses (error.UnsupportedConfiguration of
    src/model.zig and src/gpu_engine.zig)."""

    def __init__(self, what: str):
        RuntimeError.__init__(self, f"{what}: UnsupportedConfiguration")
        self.code = -21
        self.kind = "UnsupportedConfiguration"


class TensorInfo(C.Structure):
    _fields_ = [("name", C.c_char_p), ("rank", C.c_uint32), ("dims", C.c_uint64 * 4), ("type_id", C.c_uint32),
                ("relative_offset", C.c_uint64), ("file_offset", C.c_uint64), ("byte_length", C.c_uint64)]


_bound = False


def _lib() -> C.CDLL:
    global _bound
    L = _engine.lib()
    if not _bound:
        vp, u32, u64 = C.c_void_p, C.c_uint32, C.c_uint64
        sigs = {
            "gg_parse": ([C.c_char_p, C.c_size_t, u64, C.POINTER(vp)], C.c_int),
            "gg_open": ([C.c_char_p, C.POINTER(vp)], C.c_int),
            "gg_free": ([vp], None),
            "gg_version": ([vp], u32),
            "gg_alignment": ([vp], u32),
            "gg_data_offset": ([vp], u64),
            "gg_tensor_count": ([vp], u32),
            "gg_tensor_at": ([vp, u32, C.POINTER(TensorInfo)], C.c_int),
            "gg_find_tensor": ([vp, C.c_char_p, C.POINTER(TensorInfo)], C.c_int),
            "gg_expert_range": ([vp, C.c_char_p, u32, C.POINTER(u64), C.POINTER(u64)], C.c_int),
            "gg_is_expert_tensor": ([C.c_char_p], C.c_int),
            "gg_metadata_u64": ([vp, C.c_char_p, C.POINTER(u64)], C.c_int),
            "gg_metadata_raw": ([vp, C.c_char_p, C.POINTER(u32), C.POINTER(C.POINTER(C.c_uint8)),
                                 C.POINTER(C.c_size_t)], C.c_int),
            "gg_validate_gyro": ([vp], C.c_int),
        }
        for name, (args, res) in sigs.items():
            f = getattr(L, name)
            f.argtypes, f.restype = args, res
        _bound = True
    return L


def _check(code: int, what: str) -> None:
    if code != 0:
        raise GgufError(code, what)


@dataclass
class Tensor:
    name: str
    rank: int
    dims: tuple
    type_id: int
    file_offset: int
    byte_length: int | None


class Model:
    def __init__(self, handle: C.c_void_p):
        self._h = handle

    def close(self) -> None:
        if self._h:
            _lib().gg_free(self._h)
            self._h = None

    def __del__(self):
        self.close()

    @property
    def version(self) -> int:
        return _lib().gg_version(self._h)

    @property
    def alignment(self) -> int:
        return _lib().gg_alignment(self._h)

    @property
    def data_offset(self) -> int:
        return _lib().gg_data_offset(self._h)

    def tensors(self) -> list[Tensor]:
        L = _lib()
        out = []
        for i in range(L.gg_tensor_count(self._h)):
            t = TensorInfo()
            _check(L.gg_tensor_at(self._h, i, C.byref(t)), "gg_tensor_at")
            out.append(self._conv(t))
        return out

    @staticmethod
    def _conv(t: TensorInfo) -> Tensor:
        return Tensor(t.name.decode(), t.rank, tuple(int(d) for d in t.dims[:t.rank]), t.type_id, t.file_offset,
                      None if t.byte_length == 2 ** 64 - 1 else int(t.byte_length))

    def tensor(self, name: str) -> Tensor:
        t = TensorInfo()
        _check(_lib().gg_find_tensor(self._h, name.encode(), C.byref(t)), f"tensor {name}")
        return self._conv(t)

    def has_tensor(self, name: str) -> bool:
        t = TensorInfo()
        return _lib().gg_find_tensor(self._h, name.encode(), C.byref(t)) == 0

    def expert_range(self, name: str, expert: int) -> tuple[int, int]:
        off, n = C.c_uint64(), C.c_uint64()
        _check(_lib().gg_expert_range(self._h, name.encode(), expert, C.byref(off), C.byref(n)),
               f"expert {expert} of {name}")
        return off.value, n.value

    def metadata_u64(self, key: str) -> int:
        v = C.c_uint64()
        _check(_lib().gg_metadata_u64(self._h, key.encode(), C.byref(v)), f"metadata {key}")
        return v.value

    def has(self, key: str) -> bool:
        kind = C.c_uint32()
        return _lib().gg_metadata_raw(self._h, key.encode(), C.byref(kind), None, None) == 0

    def metadata(self, key: str):
        """A metadata value: int, float, bool, str, or a list of them (one array level)."""
        kind, raw, n = C.c_uint32(), C.POINTER(C.c_uint8)(), C.c_size_t()
        _check(_lib().gg_metadata_raw(self._h, key.encode(), C.byref(kind), C.byref(raw), C.byref(n)),
               f"metadata {key}")
        b = bytes(raw[:n.value])
        return _decode(kind.value, b, 0)[0]

    def validate_gyro(self) -> None:
        _check(_lib().gg_validate_gyro(self._h), "validate_gyro")


_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 10: "<Q", 11: "<q", 12: "<d"}


def _decode(kind: int, b: bytes, pos: int):
    """Value of GGUF type `kind` at b[pos:] (src/gguf.zig:13-17) and the position after it."""
    import struct
    if kind in _SCALAR:
        fmt = _SCALAR[kind]
        return struct.unpack_from(fmt, b, pos)[0], pos + struct.calcsize(fmt)
    if kind == 7:
        return b[pos] == 1, pos + 1
    if kind == 8:
        (n,) = struct.unpack_from("<Q", b, pos)
        return b[pos + 8:pos + 8 + n].decode(), pos + 8 + n
    et, n = struct.unpack_from("<IQ", b, pos)
    pos += 12
    out = []
    for _ in range(n):
        v, pos = _decode(et, b, pos)
        out.append(v)
    return out, pos


def parse(prefix: bytes, file_size: int) -> Model:
    h = C.c_void_p()
    _check(_lib().gg_parse(prefix, len(prefix), file_size, C.byref(h)), "gg_parse")
    return Model(h)


def open_model(path: str) -> Model:
    h = C.c_void_p()
    _check(_lib().gg_open(str(path).encode(), C.byref(h)), f"gg_open {path}")
    return Model(h)


def is_expert_tensor(name: str) -> bool:
    return bool(_lib().gg_is_expert_tensor(name.encode()))


def load_layer_experts(path: str, layer: int) -> dict:
    """Expert matrices of layer `layer` as read-only views of the mapped file: gate, up, down
    (lists over experts of [rows, row bytes] uint8 arrays), types [n_expert, 3], E, F, n_expert."""
    m = open_model(path)
    try:
        names = [f"blk.{layer}.ffn_{p}_exps.weight" for p in ("gate", "up", "down")]
        ts = [m.tensor(n) for n in names]
        for t in ts:
            if t.type_id not in GYRO_BLOCK_BYTES or t.rank != 3:
                raise GgufError(-14, t.name)
        E, F, NE = ts[0].dims
        if ts[1].dims != (E, F, NE) or ts[2].dims != (F, E, NE):
            raise GgufError(-9, "expert tensor shapes")
        mm = np.memmap(path, dtype=np.uint8, mode="r")
        out = {"E": E, "F": F, "n_expert": NE, "gate": [], "up": [], "down": [],
               "types": np.array([[t.type_id for t in ts]] * NE, np.uint32)}
        for key, t, rows, cols in (("gate", ts[0], F, E), ("up", ts[1], F, E), ("down", ts[2], E, F)):
            row_bytes = cols // 128 * GYRO_BLOCK_BYTES[t.type_id]
            for e in range(NE):
                off, n = m.expert_range(t.name, e)
                assert n == rows * row_bytes
                out[key].append(mm[off:off + n].reshape(rows, row_bytes))
        return out
    finally:
        m.close()


def _rotation(m: "Model"):
    """The released rotation metadata as the model loader reads it (src/model.zig:299-323): the
    listed weight names, the sign widths and values; the block size must be 128
    (src/model.zig:312) and every listed name an expert projection (src/model.zig:421-429)."""
    for key in ("prism.hadamard.weight_names", "prism.hadamard.sign_widths", "prism.hadamard.sign_values",
                "prism.hadamard.block_size"):
        if not m.has(key):
            raise GgufError(-18, key)
    if int(m.metadata("prism.hadamard.block_size")) != 128:
        raise UnsupportedConfiguration("prism.hadamard.block_size must be 128")
    names = list(m.metadata("prism.hadamard.weight_names"))
    for n in names:
        if not n.endswith((".ffn_gate_exps.weight", ".ffn_up_exps.weight", ".ffn_down_exps.weight")):
            raise UnsupportedConfiguration(f"prism.hadamard lists {n}, which this graph does not rotate")
    return names, list(m.metadata("prism.hadamard.sign_widths")), list(m.metadata("prism.hadamard.sign_values"))


def load_layer(path: str, layer: int):
    """One MoE layer of a GGUF file as a gyrodx.synth.Layer for gm_add_layer: the routed experts
    (load_layer_experts), the fp32 router "blk.<l>.ffn_gate_inp.weight" (E x n_expert),
    n_used and the optional expert-weights scale from "<arch>.expert_used_count" /
    "<arch>.expert_weights_scale" (src/model.zig:262-285), and the explicit Hadamard signs of the
    gate and down inputs: a tensor listed in prism.hadamard.weight_names takes the run of
    prism.hadamard.sign_values that belongs to its input width (src/model.zig:306-333). The
    rotation metadata is validated first (src/gguf.zig:182-250), and refused as the loaders refuse
    it: a block size other than 128 (src/model.zig:312), a listed tensor that is not an expert
    projection (src/model.zig:421-429), or up-projection signs that are not the gate's
    (src/gpu_engine.zig:404). The shared expert, when the file has one
    ("blk.<l>.ffn_{gate,up,down}_shexp.weight" in bf16, Q8_0 or fp32, and the fp32
    "blk.<l>.ffn_gate_inp_shexp.weight", src/model.zig:413-416), is read as well."""
    from .synth import Layer
    m = open_model(path)
    try:
        m.validate_gyro()
        names, widths, values = _rotation(m)
        arch = m.metadata("general.architecture")
        n_used = int(m.metadata(f"{arch}.expert_used_count"))
        scale = float(m.metadata(f"{arch}.expert_weights_scale")) if m.has(f"{arch}.expert_weights_scale") else 0.0
        r = m.tensor(f"blk.{layer}.ffn_gate_inp.weight")
        if r.type_id != 0 or r.rank != 2:
            raise GgufError(-14, r.name)
        E, NE = r.dims
        mm = np.memmap(path, dtype=np.uint8, mode="r")
        router = np.frombuffer(mm[r.file_offset:r.file_offset + r.byte_length], np.float32).reshape(NE, E)

        def signs(name: str, width: int):
            """(offset into sign_values, signs) of a listed tensor, None when it is not listed."""
            if name not in names:
                return None
            off = 0
            for w in widths:
                if w == width:
                    return off, np.asarray(values[off:off + w], np.float32)
                off += w
            raise UnsupportedConfiguration(f"no signs of width {width} for {name}")

        F = m.tensor(f"blk.{layer}.ffn_down_exps.weight").dims[0]
        gs = signs(f"blk.{layer}.ffn_gate_exps.weight", E)
        us = signs(f"blk.{layer}.ffn_up_exps.weight", E)
        ds = signs(f"blk.{layer}.ffn_down_exps.weight", F)
        # The gate and up products share one rotated input (src/gpu_engine.zig:404).
        if us is not None and (gs is None or us[0] != gs[0]):
            raise UnsupportedConfiguration("up-projection signs differ from the gate's")
        shared = _shared_expert(m, mm, layer, E)
    finally:
        m.close()
    ex = load_layer_experts(path, layer)
    if ex["E"] != E or ex["n_expert"] != NE or ex["F"] != F:
        raise GgufError(-9, "router and expert shapes")
    L = Layer(E=E, F=ex["F"], n_expert=NE, n_used=n_used, types=ex["types"], gate=ex["gate"], up=ex["up"],
              down=ex["down"], router=np.ascontiguousarray(router), router_bias=None,
              gate_signs=None if gs is None else gs[1], down_signs=None if ds is None else ds[1],
              expert_weights_scale=scale)
    if shared is not None:
        L.SF, L.sh_type, L.sh_gate, L.sh_up, L.sh_down, L.sh_gate_inp = shared
    return L


# GGML tensor types of the shared expert's matrices that the engine accepts (src/kernels.zig:7-10)
# and their row bytes for `cols` columns.
SHARED_TYPES = {0: lambda c: c * 4, 30: lambda c: c * 2, 8: lambda c: c // 32 * 34}


def _shared_expert(m: "Model", mm, layer: int, E: int):
    """(SF, type, gate, up, down, gate_inp) of the layer's shared expert, or None when the file
    has none: gate and up [SF rows of E columns], down [E rows of SF columns] as raw row bytes of
    one GGML type (fp32, bf16 or Q8_0), gate_inp fp32 [E]."""
    names = [f"blk.{layer}.ffn_{p}_shexp.weight" for p in ("gate", "up", "down")]
    if not all(m.has_tensor(n) for n in names):
        return None
    ts = [m.tensor(n) for n in names]
    ty = ts[0].type_id
    if any(t.type_id != ty or t.rank != 2 for t in ts) or ty not in SHARED_TYPES:
        raise GgufError(-14, names[0])
    if ts[0].dims[0] != E or ts[1].dims != ts[0].dims:
        raise GgufError(-9, "shared expert gate/up shape")
    SF = ts[0].dims[1]
    if ts[2].dims != (SF, E):
        raise GgufError(-9, "shared expert down shape")
    if ty == 8 and (E % 32 or SF % 32):
        raise GgufError(-9, "Q8_0 rows need a multiple of 32 columns")

    def rows(t, n_rows, cols):
        rb = SHARED_TYPES[ty](cols)
        if t.byte_length != n_rows * rb:
            raise GgufError(-9, t.name)
        return np.array(mm[t.file_offset:t.file_offset + t.byte_length]).reshape(n_rows, rb)

    gi = m.tensor(f"blk.{layer}.ffn_gate_inp_shexp.weight")
    if gi.type_id != 0 or gi.rank != 1 or gi.dims[0] != E:
        raise GgufError(-14, gi.name)
    gate_inp = np.frombuffer(mm[gi.file_offset:gi.file_offset + gi.byte_length], np.float32).copy()
    return SF, ty, rows(ts[0], SF, E), rows(ts[1], SF, E), rows(ts[2], E, SF), gate_inp
