"""The conformance commands on the GPU (src/native.zig:72-152): `gyro` validates the device
decoder against the CPU decoder for all eight types with zero error, and `stream` reads an
expert's gate, up and down slices of a written model file into device memory and back,
equal to the file's bytes."""
import json

import pytest

from gguf_fixture import write_layer_file
from gyrodx import KERNEL_DIR, commands, synth

pytestmark = pytest.mark.gpu


def test_gyro_command(capsys):
    recs = commands.validate_gyro(str(KERNEL_DIR / "gyro_decode.co"))
    assert [r["type_id"] for r in recs] == list(range(144, 152))
    assert all(r["validation_passed"] and r["max_absolute_error"] == 0.0 and r["values"] == 8192 for r in recs)
    assert commands.main(["gyro", str(KERNEL_DIR / "gyro_decode.co")]) == 0
    assert '"type_name": "TQK4"' in capsys.readouterr().out


def test_stream_command(tmp_path, capsys):
    layer = synth.make_layer(4, E=1024, F=512, n_expert=8, n_used=2, type_id=148)
    path = tmp_path / "m.gguf"
    write_layer_file(path, layer, arch="qwen4exp")
    for expert in (0, 7):
        rec = commands.stream(str(path), 0, expert)
        print(f"stream expert {expert}: {rec}", flush=True)
        assert rec["readback_equal"] and not rec["expert_compute_executed"]
    capsys.readouterr()
    assert commands.main(["stream", str(path), "0", "3"]) == 0
    rec = json.loads(capsys.readouterr().out)
    assert rec["expert"] == 3 and rec["bytes"] == 3 * 512 * 1024 // 128 * 50
