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
             -16: "InvalidMetadata", -17: "IO", -18: "NotFound"}

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
