"""Per-lane scratch memory and pipeline names of the built kernels, read from their code objects.

A kernel that spills registers or places a local array in scratch memory runs its loads and
stores through the scratch path; a decode kernel did so once after an unrelated edit and ran
2.3x slower with unchanged outputs, which no parity test can see. This test reads the AMDGPU
metadata (msgpack) of every built code object and checks `.private_segment_fixed_size`, and
reads the `gd_entry` and `gd_workgroup` globals through which the runtime loads each kernel.
Runs on the CPU; skipped when the kernels are not built.
"""
import struct
from pathlib import Path

import pytest

KERNELS = Path(__file__).resolve().parents[1] / "gyro-dx_amd" / "build" / "kernels"

# Kernels whose scratch use is known and measured: the persistent TQ2_T GEMMs spill a few
# registers at unit boundaries (two groups per CU hold them to 128 VGPRs).
ALLOWED = {"moe_prefill_gemm": 32, "moe_prefill_gemm_s": 72}


def _msgpack_uint(buf: bytes, i: int) -> int:
    b = buf[i]
    if b < 0x80:
        return b
    if b == 0xCC:
        return buf[i + 1]
    if b == 0xCD:
        return int.from_bytes(buf[i + 1:i + 3], "big")
    if b == 0xCE:
        return int.from_bytes(buf[i + 1:i + 5], "big")
    raise ValueError(f"not a msgpack unsigned integer: 0x{b:02x}")


def _meta_uint(blob: bytes, key: str) -> int:
    k = key.encode()
    i = blob.find(k)
    assert i >= 0, f"{key} not in the code object's metadata"
    assert blob.find(k, i + 1) < 0, f"more than one kernel in the code object ({key} twice)"
    return _msgpack_uint(blob, i + len(k))


def _gfx_elf(blob: bytes) -> bytes:
    """The gfx950 ELF of a code object: the file itself, or its entry of a clang offload bundle
    (magic, u64 entry count, then per entry u64 offset, u64 size, u64 id length, id)."""
    if blob.startswith(b"\x7fELF"):
        return blob
    assert blob.startswith(b"__CLANG_OFFLOAD_BUNDLE__")
    n = struct.unpack_from("<Q", blob, 24)[0]
    pos = 32
    for _ in range(n):
        off, size, idlen = struct.unpack_from("<QQQ", blob, pos)
        ident = blob[pos + 24:pos + 24 + idlen]
        pos += 24 + idlen
        if b"gfx950" in ident:
            return blob[off:off + size]
    raise AssertionError("no gfx950 entry in the bundle")


def _elf_global(elf: bytes, name: str, size: int) -> bytes:
    """The initial bytes of global `name` (a symbol of .symtab) in an ELF64 little-endian object."""
    assert elf[:4] == b"\x7fELF" and elf[4] == 2 and elf[5] == 1
    shoff, = struct.unpack_from("<Q", elf, 0x28)
    shentsize, shnum = struct.unpack_from("<HH", elf, 0x3A)
    secs = [struct.unpack_from("<IIQQQQIIQQ", elf, shoff + i * shentsize) for i in range(shnum)]
    # (name, type, flags, addr, offset, size, link, info, addralign, entsize)
    for sec in secs:
        if sec[1] != 2:  # SHT_SYMTAB
            continue
        strtab = secs[sec[6]]
        for i in range(sec[5] // 24):
            st_name, st_info, st_other, st_shndx, st_value, st_size = struct.unpack_from("<IBBHQQ", elf, sec[4] + 24 * i)
            end = elf.index(b"\0", strtab[4] + st_name)
            if elf[strtab[4] + st_name:end].decode() == name:
                assert st_size == size, (name, st_size)
                tgt = secs[st_shndx]
                start = tgt[4] + st_value - tgt[3]
                return elf[start:start + size]
    raise AssertionError(f"{name} not in the symbol table")


def _objects():
    return sorted(KERNELS.glob("*.co")) if KERNELS.is_dir() else []


@pytest.mark.skipif(not _objects(), reason="kernels not built")
@pytest.mark.parametrize("co", _objects(), ids=lambda p: p.stem)
def test_kernel_scratch(co):
    blob = co.read_bytes()
    assert blob.startswith(b"__CLANG_OFFLOAD_BUNDLE__") or blob.startswith(b"\x7fELF")
    scratch = _meta_uint(blob, ".private_segment_fixed_size")
    limit = ALLOWED.get(co.stem, 0)
    assert scratch <= limit, f"{co.stem} uses {scratch} bytes of scratch per lane (allowed {limit})"


def test_msgpack_uint_forms():
    assert _msgpack_uint(bytes([0x1C]), 0) == 28
    assert _msgpack_uint(bytes([0xCC, 0xD3]), 0) == 211
    assert _msgpack_uint(bytes([0xCD, 0x01, 0x00]), 0) == 256
    assert _msgpack_uint(bytes([0xCE, 0, 0, 1, 0]), 0) == 256
    with pytest.raises(ValueError):
        _msgpack_uint(bytes([0xA0]), 0)


@pytest.mark.skipif(not _objects(), reason="kernels not built")
@pytest.mark.parametrize("co", _objects(), ids=lambda p: p.stem)
def test_kernel_entry_names_its_file(co):
    """gd_create_pipeline finds the kernel through the module's 32-byte gd_entry string and its
    workgroup size through gd_workgroup; the engine names each pipeline by its file. A kernel
    defined through a macro argument must expand the name before it is stringised."""
    elf = _gfx_elf(co.read_bytes())
    entry = _elf_global(elf, "gd_entry", 32).rstrip(b"\0").decode()
    assert entry == co.stem
    wg = struct.unpack("<3I", _elf_global(elf, "gd_workgroup", 12))
    assert all(wg) and wg[0] * wg[1] * wg[2] <= 1024
