"""The C-ABI libraries load and export every entry point their headers declare (CPU only; no
compute calls). Struct layouts match src/native_abi.zig:87-95."""
import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
BUILD = ROOT / "gyro-dx_amd" / "build"


def declared(header, prefix):
    """Function declarations: `<API macro> <return type> <name>(`."""
    text = (ROOT / "include" / header).read_text()
    return sorted(set(re.findall(rf"\b(?:GD|GM|GG)_API\s+[\w ]+?\*?\s*\b({prefix}[a-z0-9_]+)\s*\(", text)))


def exported(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib)], capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


@pytest.mark.parametrize("lib,header,prefix,count", [
    ("libgyro_native.so", "gyro_native.h", "gd_", 29),
    ("libgyro_moe.so", "gyro_moe.h", "gm_", 17),
    ("libgyro_moe.so", "gyro_gguf.h", "gg_", 14),
])
def test_exports(lib, header, prefix, count):
    path = BUILD / lib
    assert path.exists(), f"{path} not built"
    names = declared(header, prefix)
    assert len(names) == count, names
    missing = set(names) - exported(path)
    assert not missing, missing
    C.CDLL(str(path))  # loads (resolves libamdhip64) without a GPU


def test_native_binding_lists_every_symbol():
    from gyrodx import native
    assert sorted(native.SYMBOLS) == declared("gyro_native.h", "gd_")


def test_struct_layouts():
    from gyrodx import native
    assert C.sizeof(native.Options) == 20
    assert C.sizeof(native.Caps) == 184
    assert native.Caps.adapter_name.offset == 56
    assert C.sizeof(native.Range) == 24
    assert C.sizeof(native.BufferInfo) == 32
    assert native.BufferInfo.mapped.offset == 8


def test_kernels_built():
    kernels = {p.stem for p in (BUILD / "kernels").glob("*.co")}
    reference = {"mv_f32", "mv_bf16", "mv_q8", "q8_repack", "moe_route", "moe_resolve", "moe_gyro", "moe_act", "rotate128",
                 "moe_combine", "ew", "gyro_decode", "linalg_smoke", "moe_gyro_x"}
    fast = {"moe_router", "moe_decode_gu", "moe_decode_gu_b", "moe_decode_down", "moe_dequant", "moe_prefill_router", "moe_prefill_router_w",
            "moe_prefill_topk", "moe_prefill_sort", "moe_prefill_gu", "moe_prefill_down", "moe_prefill_combine",
            "moe_stack_norm", "moe_decode_gu_x", "moe_decode_gu_xb", "moe_decode_down_x", "moe_decode_down_xb", "moe_decode_down_g", "moe_decode_gu_g", "moe_decode_gu_xg", "moe_decode_down_xg", "moe_prefill_gu_x", "moe_prefill_down_x", "gd_table_set"}
    assert reference | fast <= kernels, (reference | fast) - kernels
