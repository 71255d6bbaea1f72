"""The reference's hardware-conformance commands on the MI355X (src/native.zig:72-152):

- `gyro CODE [adapter]` (validateGyro): for each of the eight Gyro types, 64 blocks of LCG
  bytes (seed 0x4759524f) with twelve edge scales are decoded on the CPU by `decode_row` and by
  the device decoder in CODE through gd_validate_gyro, which requires bit equality; one JSON
  record per type.
- `stream MODEL LAYER EXPERT [adapter]` (stream): the expert's gate, up and down slices
  (src/plan.zig:17-31) are read from the file into a device buffer by gd_read_ranges, read back
  and compared with the file's bytes; one JSON record. No expert product runs.

Run as `python -m gyrodx.commands gyro build/kernels/gyro_decode.co` or
`python -m gyrodx.commands stream model.gguf 0 5`.
"""
from __future__ import annotations

import ctypes as C
import json
import os
import sys

import numpy as np

from . import CODEBOOK, gguf, native

TIMEOUT_MS = 30000
# src/gyro.zig:32-41: type id -> (bits per step k, steps per block, block bytes).
TYPES = {144: (8, 32, 34), 145: (6, 32, 26), 146: (7, 32, 30), 147: (5, 64, 42), 148: (6, 64, 50),
         149: (7, 64, 58), 150: (5, 32, 22), 151: (4, 32, 18)}
# The type table's names (src/gyro.zig:33-40), printed by validateGyro as info.name.
TYPE_NAMES = {144: "TQ2_T", 145: "TQK6", 146: "TQK7", 147: "TQP5", 148: "TQP6", 149: "TQP7", 150: "TQK5",
              151: "TQK4"}
EDGE_SCALES = (0, 0x8000, 1, 0x8001, 0x3FF, 0x83FF, 0x400, 0x8400, 0x3C00, 0xBC00, 0x7BFF, 0xFBFF)


class CommandError(RuntimeError):
    pass


def decode_row(type_id: int, src: np.ndarray, codebook: bytes) -> np.ndarray:
    """Strict CPU decode of Gyro blocks (src/gyro.zig:81-117), vectorised over blocks: the
    trellis state of each step (TQ2_T: byte pair (step + 31) % 32, step; other types: the k-bit
    window ending at bit (steps - 1 - step) k of the circular stream, 16 bits wide), its low
    15 bits hashed by 0x9e3779b1, one (steps 64) or two (steps 32) 11-bit codebook pair
    indices from the hash's top bits, each value fp32(scale) * fp32(codebook), one rounding."""
    k, steps, bb = TYPES[type_id]
    blocks = np.ascontiguousarray(src, np.uint8).reshape(-1, bb)
    scale = blocks[:, :2].copy().view(np.float16).astype(np.float32)[:, 0]
    stream = blocks[:, 2:].astype(np.uint32)
    n = bb - 2
    step = np.arange(steps)
    if type_id == 144:
        state = (stream[:, (step + 31) % 32] << 8) | stream[:, step]
    else:
        off = (steps - 1 - step) * k
        byte = off >> 3
        word = stream[:, byte] | (stream[:, (byte + 1) % n] << 8) | (stream[:, (byte + 2) % n] << 16)
        state = (word >> (off & 7).astype(np.uint32)) & 0xFFFF
    h = ((state & 0x7FFF).astype(np.uint64) * 0x9E3779B1) & 0xFFFFFFFF
    book = np.frombuffer(codebook, np.float16).astype(np.float32).reshape(2048, 2)
    idx = (h >> 21)[:, :, None] if steps == 64 else np.stack([h >> 21, (h >> 10) & 2047], axis=2)
    vals = book[idx.astype(np.int64)]  # [blocks, steps, pairs, 2]
    return (scale[:, None, None, None] * vals).astype(np.float32).reshape(-1)


def recipe_blocks(type_id: int, state: int) -> tuple[np.ndarray, int]:
    """64 blocks of LCG bytes (state = state * 1664525 + 1013904223, byte = state >> 24) with
    EDGE_SCALES[block % 12] as each block's scale (src/native.zig:127-140)."""
    bb = TYPES[type_id][2]
    enc = np.empty(bb * 64, np.uint8)
    for i in range(enc.size):
        state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
        enc[i] = state >> 24
    for b in range(64):
        enc[b * bb:b * bb + 2] = np.array([EDGE_SCALES[b % 12]], np.uint16).view(np.uint8)
    return enc, state


def _context(adapter: int):
    opts = native.Options(adapter, 0, 0, 32 << 20, 1024)
    h = C.c_void_p()
    native.check(native.lib().gd_create(C.byref(opts), C.byref(h)), "gd_create")
    return h


def validate_gyro(code_path: str, adapter: int = 0) -> list[dict]:
    code = open(code_path, "rb").read()
    book = CODEBOOK.read_bytes()
    L = native.lib()
    ctx = _context(adapter)
    out, state = [], 0x4759524F
    try:
        for type_id in range(144, 152):
            enc, state = recipe_blocks(type_id, state)
            expected = decode_row(type_id, enc, book)
            err = C.c_float()
            native.check(L.gd_validate_gyro(ctx, code, len(code), book, len(book), enc.ctypes.data, enc.size, type_id,
                                            expected.ctypes.data, expected.size, C.byref(err), TIMEOUT_MS),
                         f"gd_validate_gyro type {type_id}")
            out.append({"type_id": type_id, "type_name": TYPE_NAMES[type_id], "blocks": 64, "values": int(expected.size),
                        "max_absolute_error": float(err.value), "validation_passed": True})
    finally:
        native.check(L.gd_destroy(ctx, TIMEOUT_MS), "gd_destroy")
    return out


def expert_bundle(m: gguf.Model, layer: int, expert: int) -> list[tuple[int, int]]:
    """(file offset, bytes) of the expert's gate, up and down slices (src/plan.zig:17-31)."""
    if m.metadata("general.architecture") != "qwen4exp":
        raise CommandError("UnsupportedArchitecture")
    if layer >= m.metadata_u64("qwen4exp.block_count"):
        raise CommandError("InvalidExpert")
    out = []
    for kind in ("gate", "up", "down"):
        name = f"blk.{layer}.ffn_{kind}_exps.weight"
        try:
            t = m.tensor(name)
        except gguf.GgufError:
            raise CommandError("IncompleteExpertSet") from None
        if t.rank != 3 or t.dims[2] != m.metadata_u64("qwen4exp.expert_count"):
            raise CommandError("IncompleteExpertSet")
        out.append(m.expert_range(name, expert))
    return out


def stream(model_path: str, layer: int, expert: int, adapter: int = 0) -> dict:
    m = gguf.open_model(model_path)
    try:
        bundle = expert_bundle(m, layer, expert)
    finally:
        m.close()
    ranges, total = (native.Range * 3)(), 0
    for i, (off, n) in enumerate(bundle):
        if n > 32 << 20:
            raise CommandError("ExpertProjectionTooLarge")
        ranges[i] = native.Range(off, total, n, 0)
        total += n
    if total > 0xFFFFFFFF:
        raise CommandError("ExpertBundleTooLarge")
    L = native.lib()
    ctx = _context(adapter)
    fh, buf = C.c_void_p(), C.c_void_p()
    try:
        native.check(L.gd_open_file(ctx, os.fsencode(model_path), C.byref(fh)), "gd_open_file")
        size = C.c_uint64()
        native.check(L.gd_file_size(fh, C.byref(size)), "gd_file_size")
        if size.value != os.path.getsize(model_path):
            raise CommandError("ModelChanged")
        native.check(L.gd_create_buffer(ctx, total, C.byref(buf)), "gd_create_buffer")
        ticket = C.c_uint64()
        native.check(L.gd_read_ranges(ctx, fh, buf, ranges, 3, C.byref(ticket)), "gd_read_ranges")
        native.check(L.gd_wait_storage(ctx, ticket, TIMEOUT_MS), "gd_wait_storage")
        actual = np.empty(total, np.uint8)
        native.check(L.gd_readback(ctx, buf, 0, total, actual.ctypes.data, TIMEOUT_MS), "gd_readback")
        with open(model_path, "rb") as f:
            expected = b"".join(os.pread(f.fileno(), n, off) for off, n in bundle)
        if len(expected) != total:
            raise CommandError("UnexpectedEnd")
        if actual.tobytes() != expected:
            raise CommandError("TransferMismatch")
        return {"layer": layer, "expert": expert, "bytes": total, "storage_ticket": ticket.value,
                "readback_equal": True, "expert_compute_executed": False}
    finally:
        if buf:
            native.check(L.gd_release_buffer(ctx, buf, TIMEOUT_MS), "gd_release_buffer")
        if fh:
            native.check(L.gd_release_file(ctx, fh, TIMEOUT_MS), "gd_release_file")
        native.check(L.gd_destroy(ctx, TIMEOUT_MS), "gd_destroy")


def main(argv: list[str]) -> int:
    if len(argv) >= 2 and argv[0] == "gyro" and len(argv) <= 3:
        for rec in validate_gyro(argv[1], int(argv[2]) if len(argv) > 2 else 0):
            print(json.dumps(rec, indent=2))
        return 0
    if len(argv) >= 4 and argv[0] == "stream" and len(argv) <= 5:
        print(json.dumps(stream(argv[1], int(argv[2]), int(argv[3]), int(argv[4]) if len(argv) > 4 else 0), indent=2))
        return 0
    print("usage: gyro CODE [adapter] | stream MODEL LAYER EXPERT [adapter]", file=sys.stderr)
    return 2


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
