"""Per-lane scratch memory of the built kernels, read from their code-object metadata.

A kernel that spills registers or places a local array in scratch memory runs its loads and
stores through the scratch path; a decode kernel did so once after an unrelated edit and ran
2.3x slower with unchanged outputs, which no parity test can see. This test reads the AMDGPU
metadata (msgpack) of every built code object and checks `.private_segment_fixed_size`.
Runs on the CPU; skipped when the kernels are not built.
"""
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
