"""Python bindings of the MI355X MoE hot path (ctypes over build/libgyro_native.so and
build/libgyro_moe.so). There is no CPU fallback: importing the bindings without the built
libraries raises."""
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent.parent
BUILD_DIR = PACKAGE_DIR / "build"
KERNEL_DIR = BUILD_DIR / "kernels"
CODEBOOK = PACKAGE_DIR / "data" / "gyro_codebook.f16"
