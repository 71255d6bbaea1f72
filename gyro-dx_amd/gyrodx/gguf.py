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
             -16: "InvalidMetadata", -17: "IO", -18: "NotFound", -19: "UnsupportedGyroMetadata"}

    def __init__(self, code: int, what: str):
        self.code = code
        self.kind = self.NAMES.get(code, str(code))
        super().__init__(f"{what}: {self.kind}")


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


def load_layer(path: str, layer: int):
    """One MoE layer of a GGUF file as a gyrodx.synth.Layer for gm_add_layer: the routed experts
    (load_layer_experts), the fp32 router "blk.<l>.ffn_gate_inp.weight" (E x n_expert),
    n_used and the optional expert-weights scale from "<arch>.expert_used_count" /
    "<arch>.expert_weights_scale" (src/model.zig:262-285), and the explicit Hadamard signs of the
    gate and down inputs: a tensor listed in prism.hadamard.weight_names takes the run of
    prism.hadamard.sign_values that belongs to its input width (src/model.zig:306-333). The
    rotation metadata is validated first (src/gguf.zig:182-250)."""
    from .synth import Layer
    m = open_model(path)
    try:
        m.validate_gyro()
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
            if not m.has("prism.hadamard.weight_names") or name not in m.metadata("prism.hadamard.weight_names"):
                return None
            if m.metadata("prism.hadamard.sign_mode") != "explicit":
                return np.ones(width, np.float32)
            off = 0
            values = m.metadata("prism.hadamard.sign_values")
            for w in m.metadata("prism.hadamard.sign_widths"):
                if w == width:
                    return np.asarray(values[off:off + w], np.float32)
                off += w
            raise GgufError(-16, f"signs of width {width}")

        F = m.tensor(f"blk.{layer}.ffn_down_exps.weight").dims[0]
        gate_signs = signs(f"blk.{layer}.ffn_gate_exps.weight", E)
        down_signs = signs(f"blk.{layer}.ffn_down_exps.weight", F)
    finally:
        m.close()
    ex = load_layer_experts(path, layer)
    if ex["E"] != E or ex["n_expert"] != NE or ex["F"] != F:
        raise GgufError(-9, "router and expert shapes")
    return Layer(E=E, F=ex["F"], n_expert=NE, n_used=n_used, types=ex["types"], gate=ex["gate"], up=ex["up"],
                 down=ex["down"], router=np.ascontiguousarray(router), router_bias=None, gate_signs=gate_signs,
                 down_signs=down_signs, expert_weights_scale=scale)
