"""Seeded synthetic MoE layers in the reference's on-disk expert format.

Every array comes from numpy's PCG64 generator with a documented seed and a separate stream
per quantity, so the GPU run and the CPU baseline see the same bytes.

Expert tensors follow the GGUF layout the reference binds (src/model.zig:115-123): gate and up
are [n_expert * F rows][E columns] and down is [n_expert * E rows][F columns], each row a
sequence of Gyro blocks (src/gyro.zig:70-76). Block scales are drawn as uniform binary16 bit
patterns whose magnitude lies in [2^-8, 2^-3) with a random sign; the trellis stream bytes are
uniform random. Router weights are N(0, 0.02) fp32, activations N(0, 1), Hadamard signs
uniform +-1 (src/model.zig:305-330). An optional shared expert has N(0, 0.02) weights stored as
bf16, Q8_0 (per-32-block binary16 scale max|w| / 127, int8 quants) or fp32.
"""
from __future__ import annotations

import dataclasses
import hashlib

import numpy as np

# Gyro type table: id -> (k, steps, block_bytes), src/gyro.zig:32-41.
TYPES = {
    144: (8, 32, 34), 145: (6, 32, 26), 146: (7, 32, 30), 147: (5, 64, 42),
    148: (6, 64, 50), 149: (7, 64, 58), 150: (5, 32, 22), 151: (4, 32, 18),
}
TQ2_T = 144

# Independent streams per quantity.
STREAM_GATE, STREAM_UP, STREAM_DOWN, STREAM_ROUTER = 1, 2, 3, 4
STREAM_SIGNS, STREAM_X, STREAM_ZIPF, STREAM_TYPES, STREAM_SHARED, STREAM_NORM = 5, 6, 7, 8, 9, 10


def row_bytes(type_id: int, cols: int) -> int:
    k, steps, bb = TYPES[type_id]
    if cols % 128:
        raise ValueError("row length must be a multiple of 128")
    return cols // 128 * bb


def rng(seed: int, stream: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64([seed, stream]))


def random_blocks(g: np.random.Generator, type_id: int, rows: int, cols: int) -> np.ndarray:
    """rows x row_bytes of packed blocks: uniform stream bytes, bounded finite scales."""
    bb = TYPES[type_id][2]
    nblk = cols // 128
    raw = g.integers(0, 256, size=(rows, nblk, bb), dtype=np.uint8)
    # Scale bits: sign random, exponent field 7..11 (2^-8 .. 2^-4 leading), mantissa uniform.
    sign = g.integers(0, 2, size=(rows, nblk), dtype=np.uint16) << 15
    expo = g.integers(7, 12, size=(rows, nblk), dtype=np.uint16) << 10
    mant = g.integers(0, 1024, size=(rows, nblk), dtype=np.uint16)
    half = sign | expo | mant
    raw[:, :, 0] = (half & 0xFF).astype(np.uint8)
    raw[:, :, 1] = (half >> 8).astype(np.uint8)
    return raw.reshape(rows, nblk * bb)


@dataclasses.dataclass
class Layer:
    """One synthetic MoE layer. Expert matrices are stored per projection as
    [n_expert, rows, row_bytes] uint8 arrays; types[e, p] gives the Gyro type of expert e,
    projection p (0 gate, 1 up, 2 down)."""
    E: int
    F: int
    n_expert: int
    n_used: int
    types: np.ndarray            # [n_expert, 3] uint32
    gate: list                   # n_expert arrays [F, row_bytes(E)]
    up: list
    down: list                   # n_expert arrays [E, row_bytes(F)]
    router: np.ndarray           # [n_expert, E] fp32
    router_bias: np.ndarray | None
    gate_signs: np.ndarray | None  # [E] fp32
    down_signs: np.ndarray | None  # [F] fp32
    expert_weights_scale: float = 0.0
    SF: int = 0
    sh_type: int = 30                  # GGML type of the shared matrices: 30 bf16, 8 Q8_0, 0 fp32
    sh_gate: np.ndarray | None = None  # [SF, row bytes(E)] (bf16: [SF, E] uint16 bits)
    sh_up: np.ndarray | None = None
    sh_down: np.ndarray | None = None  # [E, row bytes(SF)] (bf16: [E, SF] uint16 bits)
    sh_gate_inp: np.ndarray | None = None  # [E] fp32
    norm_weight: np.ndarray | None = None  # [E] fp32, RMSNorm of the layer's input in a stack
    norm_eps: float = 1e-6

    def uniform_type(self) -> int | None:
        t = np.unique(self.types)
        return int(t[0]) if t.size == 1 else None

    def expert_bytes(self, e: int) -> int:
        return self.gate[e].nbytes + self.up[e].nbytes + self.down[e].nbytes

    def digest(self) -> str:
        h = hashlib.sha256()
        for e in range(self.n_expert):
            h.update(self.gate[e].tobytes()); h.update(self.up[e].tobytes()); h.update(self.down[e].tobytes())
        h.update(self.router.tobytes())
        if self.router_bias is not None:
            h.update(self.router_bias.tobytes())
        return h.hexdigest()


def zipf_bias(seed: int, n_expert: int, s: float = 1.1, factor: float = 1.0) -> np.ndarray:
    """Per-expert router-logit bias: factor * log(Zipf(s) pmf of the expert's rank); ranks are
    assigned to experts by a seeded permutation."""
    g = rng(seed, STREAM_ZIPF)
    ranks = np.arange(1, n_expert + 1, dtype=np.float64)
    pmf = ranks ** (-s)
    pmf /= pmf.sum()
    perm = g.permutation(n_expert)
    bias = np.empty(n_expert, dtype=np.float64)
    bias[perm] = factor * np.log(pmf)
    return bias.astype(np.float32)


def q8_0_quantize(w: np.ndarray) -> np.ndarray:
    """fp32 rows [rows, cols] to GGUF Q8_0 rows [rows, cols / 32 * 34]: per 32-block a binary16
    scale d = max|w| / 127 and int8 quants round(w / d)."""
    rows, cols = w.shape
    b = w.reshape(rows, cols // 32, 32).astype(np.float32)
    d = (np.abs(b).max(axis=2) / 127.0).astype(np.float16)
    df = d.astype(np.float32)
    q = np.clip(np.rint(np.divide(b, df[:, :, None], out=np.zeros_like(b), where=df[:, :, None] != 0)),
                -127, 127).astype(np.int8)
    out = np.empty((rows, cols // 32, 34), np.uint8)
    out[:, :, :2] = d.view(np.uint8).reshape(rows, cols // 32, 2)
    out[:, :, 2:] = q.view(np.uint8)
    return out.reshape(rows, cols // 32 * 34)


def make_layer(seed: int, E: int = 2048, F: int = 512, n_expert: int = 256, n_used: int = 8,
               type_id: int | None = TQ2_T, mixed_types: bool = False, zipf: float | None = None,
               zipf_factor: float = 1.0, signs: bool = True, SF: int = 0, sh_type: int = 30) -> Layer:
    if mixed_types:
        types = rng(seed, STREAM_TYPES).choice(np.array(sorted(TYPES), dtype=np.uint32),
                                               size=(n_expert, 3))
    else:
        types = np.full((n_expert, 3), type_id, dtype=np.uint32)
    gg, gu, gd = rng(seed, STREAM_GATE), rng(seed, STREAM_UP), rng(seed, STREAM_DOWN)
    gate = [random_blocks(gg, int(types[e, 0]), F, E) for e in range(n_expert)]
    up = [random_blocks(gu, int(types[e, 1]), F, E) for e in range(n_expert)]
    down = [random_blocks(gd, int(types[e, 2]), E, F) for e in range(n_expert)]
    router = (rng(seed, STREAM_ROUTER).standard_normal((n_expert, E)) * 0.02).astype(np.float32)
    gs = ds = None
    if signs:
        sg = rng(seed, STREAM_SIGNS)
        gs = (sg.integers(0, 2, E) * 2 - 1).astype(np.float32)
        ds = (sg.integers(0, 2, F) * 2 - 1).astype(np.float32)
    bias = zipf_bias(seed, n_expert, zipf, zipf_factor) if zipf else None
    layer = Layer(E=E, F=F, n_expert=n_expert, n_used=n_used, types=types.astype(np.uint32),
                  gate=gate, up=up, down=down, router=router, router_bias=bias,
                  gate_signs=gs, down_signs=ds)
    if SF:
        sh = rng(seed, STREAM_SHARED)
        def bf16(a):
            u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
            return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
        conv = {30: bf16, 8: q8_0_quantize,
                0: lambda a: np.ascontiguousarray(a, np.float32).view(np.uint8).reshape(a.shape[0], -1)}[sh_type]
        layer.SF = SF
        layer.sh_type = sh_type
        layer.sh_gate = conv((sh.standard_normal((SF, E)) * 0.02).astype(np.float32))
        layer.sh_up = conv((sh.standard_normal((SF, E)) * 0.02).astype(np.float32))
        layer.sh_down = conv((sh.standard_normal((E, SF)) * 0.02).astype(np.float32))
        layer.sh_gate_inp = (sh.standard_normal(E) * 0.02).astype(np.float32)
    return layer


def make_stack(seed: int, n_layers: int, **kw) -> list:
    """n_layers layers seeded seed, seed + 1, ...; each with RMSNorm weights 1 + 0.1 N(0, 1)."""
    layers = []
    for l in range(n_layers):
        L = make_layer(seed + l, **kw)
        L.norm_weight = (1.0 + 0.1 * rng(seed + l, STREAM_NORM).standard_normal(L.E)).astype(np.float32)
        layers.append(L)
    return layers


def make_tokens(seed: int, n: int, E: int = 2048, bf16: bool = False, stream: int = STREAM_X) -> np.ndarray:
    """n x E activations N(0, 1) in fp32; with bf16=True the values are rounded to bf16
    (round to nearest even) and returned as exactly representable fp32."""
    x = rng(seed, stream).standard_normal((n, E)).astype(np.float32)
    if bf16:
        u = x.view(np.uint32)
        u = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
        x = u.view(np.float32)
    return x
