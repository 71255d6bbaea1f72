"""The Zig dispatch snippets of INTEGRATION.md, replayed as written through the raw gd C ABI.

Every ```zig block of the document that dispatches kernels is parsed from the text (kernel name,
constant list, grid) and evaluated with the document's own names bound: buffers are gd resources
in device memory (the layer uploaded through a mapped staging resource and the `ew` copy kernel,
as src/gpu_engine.zig:447-461 uploads the codebook), scalars are the layer's shape and the sizes
the document's rules give (parts, rpg, R, S, tiles, the power-of-two scales of the shared
expert's binary16 copies). Each sequence runs as one gd_begin / gd_dispatch ... / gd_submit on
the reference's entry points (native/include/gyro_native.h); the output, ids and weights come
back through gd_readback and must equal bit for bit what gm_forward gives for the same layer and
tokens on the same path, and lie within relative RMS 2e-3 and cosine 0.9999 of the CPU oracle
(src/engine.zig:520-653), with the oracle's ids for every token whose U-th and (U+1)-th router
probabilities are separated by more than 1e-5 relative.

The CPU test checks that every snippet parses and evaluates to u32 constants and legal grids on
every case below, that each names a kernel this repository builds, and that every kernel the
engine's decode and prefill paths dispatch is named in the document.
"""
import ctypes as C
import math
import re
import types
from pathlib import Path

import numpy as np
import pytest

from gyrodx import CODEBOOK, KERNEL_DIR, native, synth
from gyrodx.engine import PATH_DECODE, PATH_PREFILL, Engine

ROOT = Path(__file__).resolve().parents[1]
DOC = ROOT / "INTEGRATION.md"
ENGINE_SRC = ROOT / "gyro-dx_amd" / "host" / "engine.cpp"
KERNEL_SRC = ROOT / "gyro-dx_amd" / "csrc" / "kernels"
TIMEOUT = 30000
NONE = 0xFFFFFFFF
REL_RMS, COSINE = 2e-3, 0.9999
X_OFF, OUT_OFF = 64, 128  # word offsets of the input and output rows in their buffers
STAGING = 16 << 20

DISPATCH = re.compile(r"try e\.dev\.dispatch\(e\.pipes\.get\(\.(\w+)\),\s*&\.\{(.*?)\},\s*(.*?)\);", re.S)


def zig_expr(src: str) -> str:
    """A constant list or grid of the document as a Python expression: @bitCast of an f32 to its
    bits, @truncate to the low 32 bits, @max, and `/` as the integer division it is on u32."""
    src = src.replace("@bitCast(", "f32_bits(").replace("@truncate(", "low32(").replace("@max(", "max(")
    return " ".join(src.replace("/", "//").split())


def snippet_blocks():
    """The document's ```zig blocks that dispatch kernels, as lists of (kernel, constants, grid)."""
    blocks = []
    for body in re.findall(r"```zig\n(.*?)```", DOC.read_text(), re.S):
        body = re.sub(r"//[^\n]*", "", body)
        calls = [(m.group(1), zig_expr(m.group(2)), zig_expr(m.group(3))) for m in DISPATCH.finditer(body)]
        if calls:
            blocks.append(calls)
    return blocks


def block(*names):
    """The snippet that dispatches exactly `names`, in order."""
    found = [b for b in snippet_blocks() if tuple(k for k, _, _ in b) == names]
    assert len(found) == 1, f"INTEGRATION.md has {len(found)} snippets dispatching {names}"
    return found[0]


def f32_bits(v) -> int:
    return int(np.array([v], np.float32).view(np.uint32)[0])


def low32(v) -> int:
    return int(v) & 0xFFFFFFFF


def evaluate(call, ns):
    """(kernel, constants, grid) of one dispatch with the document's names bound from ns."""
    name, consts, grid = call
    env = dict(vars(ns), f32_bits=f32_bits, low32=low32, max=max)
    c = eval(f"[{consts}]", {"__builtins__": {}}, env)
    g = eval(f"({grid},)", {"__builtins__": {}}, env)
    assert all(isinstance(v, int) and 0 <= v < 1 << 32 for v in c), (name, c)
    assert len(c) <= 60, (name, len(c))
    assert len(g) == 3 and all(isinstance(v, int) and 1 <= v <= 65535 for v in g), (name, g)
    return name, c, g


# The sequences: snippet blocks by the kernels they dispatch, and how a sequence combines them.
DECODE_TQ2 = ("moe_router", "moe_decode_gu", "moe_decode_down")
DECODE_G = ("moe_decode_gu_g", "moe_decode_down_g")
DECODE_X = ("moe_router", "moe_decode_gu_x", "moe_decode_down_x")
DECODE_XG = ("moe_decode_gu_xg", "moe_decode_down_xg")
PREFILL = ("moe_prefill_router", "moe_prefill_topk", "moe_prefill_sort", "moe_prefill_gu", "moe_prefill_down",
           "moe_prefill_combine")
PREFILL_X = ("moe_prefill_gu_x", "moe_prefill_down_x")
PREFILL_SH = ("moe_prefill_router", "moe_prefill_shared", "moe_prefill_shared", "moe_prefill_combine")
PREFILL_ONE = ("moe_prefill_sort", "moe_prefill_gemm", "moe_prefill_gemm_s")
PREFILL_ONE_X = ("moe_prefill_sort", "moe_prefill_gemm_x")


def sequence(kind: str, ns):
    if kind == "decode_tq2":
        # The document's rule: moe_decode_gu_b, same constants and grid, for 2 to 8 tokens.
        router, gu, down = block(*DECODE_TQ2)
        if ns.n > 1:
            gu = ("moe_decode_gu_b",) + gu[1:]
        return [router, gu, down]
    if kind == "decode_g":
        # The document's rule: moe_decode_down_gl when n_used F / 128 > 64.
        gu, down = block(*DECODE_G)
        if ns.n_used * ns.F // 128 > 64:
            down = ("moe_decode_down_gl",) + down[1:]
        return [block(*DECODE_TQ2)[0], gu, down]
    if kind == "decode_x":
        # The document's rules for 2 to 8 tokens: moe_decode_gu_xb with the same constants and
        # grid, moe_decode_down_xb with the same constants and E / 16 groups per token.
        router, gu, down = block(*DECODE_X)
        if ns.n > 1:
            gu = ("moe_decode_gu_xb",) + gu[1:]
            down = ("moe_decode_down_xb", down[1], zig_expr("E / 16, n, 1"))
        return [router, gu, down]
    if kind == "decode_xg":
        return [block(*DECODE_TQ2)[0], *block(*DECODE_XG)]
    p = block(*PREFILL)
    if kind in ("prefill_gemm", "prefill_gemm_s"):  # the sort with the queue buffer, both GEMMs in one launch
        sort, gemm, gemm_s = block(*PREFILL_ONE)
        return [*p[:2], sort, gemm_s if kind == "prefill_gemm_s" else gemm, p[5]]
    if kind == "prefill_gemm_x":  # the type-generic pair in one launch, the sort with the queue buffer
        sort, gemm = block(*PREFILL_ONE_X)
        mid = [gemm]
        if ns.SF:
            sh = block(*PREFILL_SH)
            return [sh[0], p[1], sort, *mid, *sh[1:]]
        return [*p[:2], sort, *mid, p[5]]
    mid = block(*PREFILL_X) if ns.mixed else p[3:5]
    if ns.SF:
        sh = block(*PREFILL_SH)
        return [sh[0], *p[1:3], *mid, *sh[1:]]
    return [*p[:3], *mid, p[5]]


# kind, E, F, experts, top-k, tokens, synth.make_layer extras
CASES = [
    ("decode_tq2", 2048, 512, 64, 8, 5, {"zipf": 1.1}),
    ("decode_tq2", 1024, 512, 32, 8, 8, {"signs": False}),
    ("decode_g", 2560, 640, 64, 10, 3, {}),
    ("decode_g", 256, 1024, 32, 16, 2, {}),
    ("decode_x", 2048, 512, 64, 8, 4, {"mixed_types": True, "SF": 256}),
    ("decode_x", 1024, 512, 32, 8, 3, {"mixed_types": True, "SF": 512, "signs": False}),
    ("decode_xg", 2560, 640, 64, 10, 3, {"mixed_types": True}),
    ("decode_xg", 1024, 256, 32, 3, 5, {"mixed_types": True, "zipf": 1.1}),
    ("prefill", 1024, 512, 64, 8, 100, {}),
    ("prefill", 2560, 640, 64, 10, 70, {"zipf": 1.1}),
    ("prefill", 1024, 384, 32, 6, 50, {"mixed_types": True}),
    ("prefill", 1024, 512, 32, 8, 40, {"SF": 256}),
    ("prefill", 1024, 256, 16, 4, 30, {"mixed_types": True, "SF": 128, "signs": False}),
    ("prefill_gemm", 1024, 512, 64, 8, 100, {}),
    ("prefill_gemm", 2560, 640, 64, 10, 70, {"zipf": 1.1}),
    ("prefill_gemm_s", 2048, 512, 256, 8, 40, {}),
    ("prefill_gemm_s", 4096, 1024, 64, 6, 9, {"signs": False}),
    ("prefill_gemm_x", 1024, 384, 32, 6, 50, {"mixed_types": True}),
    ("prefill_gemm_x", 2560, 640, 64, 10, 70, {"mixed_types": True, "zipf": 1.1}),
    ("prefill_gemm_x", 1024, 256, 16, 4, 30, {"mixed_types": True, "SF": 128, "signs": False}),
]
IDS = [f"{c[0]}-E{c[1]}-F{c[2]}-x{c[3]}-top{c[4]}-n{c[5]}" + "".join(f"-{k}" for k in c[6]) for c in CASES]


def split_router_rows(w: np.ndarray) -> np.ndarray:
    """The document's router16 layout of fp32 router rows w [NE][E], as u32 words."""
    w = np.asarray(w, np.float32)
    NE, E = w.shape
    a = np.abs(w)
    mx = np.where(np.isfinite(a), a, 0).max(axis=1)
    k = np.where(mx > 0, 15 - np.frexp(mx)[1], 0).astype(np.int32)
    v = np.ldexp(w, k[:, None]).astype(np.float32)
    hi = v.astype(np.float16)
    lo = ((v - hi.astype(np.float32)) * np.float32(2048)).astype(np.float16)
    chunks = np.stack([hi.reshape(NE, E // 16, 16), lo.reshape(NE, E // 16, 16)], axis=2)  # [NE][E/16][2][16]
    unscale = np.ldexp(np.float32(1), -k).astype(np.float32)
    return np.concatenate([chunks.reshape(-1).view(np.uint32), unscale.view(np.uint32)])


def names(L, n: int, cus: int, buffer):
    """The document's names for layer L and a call of n tokens. buffer(nbytes, data) makes a
    resource (an object with .uav, .srv and .gpu) holding `data` (bytes or None) at its start."""
    E, F, NE, U, SF = L.E, L.F, L.n_expert, L.n_used, L.SF
    assert (L.gate_signs is None) == (L.down_signs is None)
    stride = (max(L.expert_bytes(e) for e in range(NE)) + 255) & ~255
    ns = types.SimpleNamespace(E=E, F=F, NE=NE, n=n, n_used=U, SF=SF, scale=L.expert_weights_scale,
                               mixed=L.uniform_type() is None, x_off=X_OFF, out_off=OUT_OFF,
                               gate_signs_off=0, down_signs_off=E, slot_stride=stride)
    # Layer: the expert arena (bundles gate | up | down at a 256-byte stride, 256 bytes of slack),
    # the expert table, router, bias, signs, codebook, shared expert.
    arena = bytearray(NE * stride + 256)
    for e in range(NE):
        o = e * stride
        for m in (L.gate[e], L.up[e], L.down[e]):
            arena[o:o + m.nbytes] = m.tobytes()
            o += m.nbytes
    l = types.SimpleNamespace()
    l.arena = buffer(len(arena), bytes(arena))
    ns.base = l.arena.gpu
    ns.proj_bytes = L.gate[0].nbytes
    xtab = np.zeros((NE, 4), np.uint64)
    for e in range(NE):
        g = ns.base + e * stride
        t = L.types[e]
        xtab[e, :3] = (g, g + L.gate[e].nbytes, g + L.gate[e].nbytes + L.up[e].nbytes)
        xtab[e, 3] = int(t[0]) | int(t[1]) << 8 | int(t[2]) << 16
    l.xtab = buffer(xtab.nbytes, xtab.tobytes())
    l.router = buffer(L.router.nbytes, L.router.tobytes())
    l.router16 = buffer(4 * (NE * E + NE), split_router_rows(L.router).tobytes())
    ns.bias_srv = buffer(NE * 4, L.router_bias.astype(np.float32).tobytes()).srv if L.router_bias is not None else NONE
    if L.gate_signs is not None:
        signs = np.concatenate([L.gate_signs, L.down_signs]).astype(np.float32)
        ns.signs_srv = buffer(signs.nbytes, signs.tobytes()).srv
    else:
        ns.signs_srv = NONE
    ns.codebook = buffer(8192, CODEBOOK.read_bytes())
    if SF:
        assert L.sh_type == 30
        gu16 = np.concatenate([L.sh_gate, L.sh_up]).view(np.uint16)  # bf16 [2 SF][E]
        l.sh_gu = buffer(gu16.nbytes, gu16.tobytes())
        l.sh_down = buffer(L.sh_down.nbytes, np.ascontiguousarray(L.sh_down).tobytes())  # bf16 [E][SF]
        l.sh_gate = buffer(E * 4, L.sh_gate_inp.astype(np.float32).tobytes())
        # Binary16 copies, each matrix scaled by 2^k with its largest |weight| in [2^14, 2^15).
        scaled, unscale = [], []
        for m in (L.sh_gate, L.sh_up, L.sh_down):
            v = (np.ascontiguousarray(m).view(np.uint16).astype(np.uint32) << 16).view(np.float32)
            k = 15 - int(np.frexp(np.float32(np.abs(v).max()))[1])
            scaled.append(np.ldexp(v, k).astype(np.float16))
            unscale.append(math.ldexp(1.0, -k))
        l.sh_gu16 = buffer(2 * SF * E * 2, np.concatenate(scaled[:2]).tobytes())
        l.sh_down16 = buffer(E * SF * 2, scaled[2].tobytes())
        ns.unscale_gate, ns.unscale_up, ns.unscale_down = unscale
    ns.l = l
    # Sizes the document's rules give.
    ns.parts = -(-E // 1024)
    total = n * U * F
    ns.rpg = max(1, min(-(-total // cus), F, 1024 // (E // 128)))
    R = max(1, E // cus)
    while R > 1 and (E % R or U * (F // 128) * 2 * ((R + 1) // 2) > 1024 or R * U > 512):
        R -= 1
    ns.R = R
    S, rt = 1, -(-n // 32) * -(-NE // 32)
    while rt * S * 2 <= 256 and E % (128 * S * 2) == 0 and S * 2 <= 16:
        S *= 2
    ns.S = S
    ns.tiles = -(-n * U // 128) + min(NE, n * U)
    ns.n_chunks = -(-n * U // 256)
    ns.hist_words = ns.n_chunks * NE
    ns.cus = cus
    ns.small_rows = 0 if E % 512 or F % 512 else (16 if E <= 2048 else (8 if E <= 4096 else 0))
    # Call buffers, each sized for nt >= n tokens (whole 64-token tiles and one more) so that no
    # kernel's tile rounding can reach past a buffer.
    nt = -(-n // 64) * 64 + 64
    sizes = dict(x=(X_OFF + nt * E) * 4, out=(OUT_OFF + nt * E) * 4, logits=16 * nt * NE * 4, xh=nt * E * 4, xh16=nt * E * 2,
                 ids=nt * U * 4, weights=nt * U * 4, gu=ns.parts * nt * U * 2 * F * 4, act=nt * U * F * 4,
                 order=nt * U * 4, meta=(1024 + 4 * (ns.tiles + 64)) * 4, act16=nt * U * F * 2,
                 down32=nt * U * E * 4, hist=(-(-nt * U // 256)) * NE * 4, sh_h=nt * 2 * max(SF, 1) * 4, sh_g=nt * 4, x16=nt * E * 2,
                 sh_a16=nt * max(SF, 1) * 2, sh_o=nt * E * 4, sched=(64 + 2 * ns.tiles + 64) * 4)
    for k, v in sizes.items():
        setattr(ns, k, buffer(v, None))
    return ns


def make_case(case):
    kind, E, F, NE, U, n, kw = case
    L = synth.make_layer(1300 + E // 128 + F // 64 + U + n, E=E, F=F, n_expert=NE, n_used=U, **kw)
    x = synth.make_tokens(1301 + n, n, E)
    return kind, L, x


def kernel_sources():
    return {p.stem for p in KERNEL_SRC.glob("*.hip")}


# -------------------------------------------------------------------------------------------------
# CPU: the snippets parse, evaluate on every case and name built kernels; the engine's fast-path
# kernels all appear in the document.

class _Fake:
    count = 0

    def __init__(self):
        _Fake.count += 2
        self.srv, self.uav, self.gpu = _Fake.count, _Fake.count + 1, 0x7F00_0000_0000 + _Fake.count * (1 << 24)


@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_snippets_evaluate(case):
    kind, L, _ = make_case(case)
    ns = names(L, case[5], 256, lambda nbytes, data: _Fake())
    calls = sequence(kind, ns)
    srcs = kernel_sources()
    for call in calls:
        name, c, g = evaluate(call, ns)
        assert name in srcs, f"{name} has no kernel source"


def test_engine_kernels_documented():
    text = DOC.read_text()
    used = set(re.findall(r'"(moe_(?:decode|prefill|router|stack)\w*)"', ENGINE_SRC.read_text()))
    assert used, "no fast-path dispatches found in the engine"
    missing = sorted(k for k in used if f"`{k}`" not in text and f".{k})" not in text)
    assert not missing, f"kernels dispatched by the engine but not named in INTEGRATION.md: {missing}"


# -------------------------------------------------------------------------------------------------
# GPU: each sequence replayed through gd_* against gm_forward and the oracle.

class Device:
    """A gd context with a mapped staging resource for uploads."""

    def __init__(self):
        self.L = native.lib()
        opts = native.Options(0, 0, 0, 32 << 20, 1024)
        self.ctx = C.c_void_p()
        native.check(self.L.gd_create(C.byref(opts), C.byref(self.ctx)), "gd_create")
        self.bufs, self.pipes = [], {}
        self.staging, self.staging_info = self._resource(STAGING, 1)

    def _resource(self, nbytes, kind):
        h, info = C.c_void_p(), native.BufferInfo()
        native.check(self.L.gd_create_resource(self.ctx, nbytes, kind, C.byref(h), C.byref(info)), "gd_create_resource")
        self.bufs.append(h)
        return h, info

    def pipe(self, name):
        if name not in self.pipes:
            code = (KERNEL_DIR / f"{name}.co").read_bytes()
            p = C.c_void_p()
            native.check(self.L.gd_create_pipeline(self.ctx, code, len(code), C.byref(p)), f"gd_create_pipeline {name}")
            self.pipes[name] = p
        return self.pipes[name]

    def run(self, calls):
        """One gd_begin .. gd_submit of (name, constants, grid) dispatches, then the wait."""
        native.check(self.L.gd_begin(self.ctx, TIMEOUT), "gd_begin")
        for name, c, g in calls:
            cst = (C.c_uint32 * len(c))(*c)
            native.check(self.L.gd_dispatch(self.ctx, self.pipe(name), cst, len(c), *g), f"gd_dispatch {name}")
        ticket = C.c_uint64()
        native.check(self.L.gd_submit(self.ctx, C.byref(ticket)), "gd_submit")
        native.check(self.L.gd_wait_compute(self.ctx, ticket, TIMEOUT), "gd_wait_compute")

    def buffer(self, nbytes, data):
        """A device resource of nbytes holding data (bytes, a multiple of 4) at its start."""
        h, info = self._resource(nbytes, 0)
        b = types.SimpleNamespace(h=h, uav=info.uav_index, srv=info.srv_index, gpu=info.gpu_address, nbytes=nbytes)
        if data:
            self.write(b, 0, data)
        return b

    def write(self, b, offset, data):
        """Copies host bytes into b at byte offset through the staging resource and `ew` (op 5:
        y = a, bit-exact) in chunks of STAGING bytes."""
        assert len(data) % 4 == 0 and offset % 4 == 0 and offset + len(data) <= b.nbytes
        for s in range(0, len(data), STAGING):
            chunk = data[s:s + STAGING]
            C.memmove(self.staging_info.mapped, chunk, len(chunk))
            words = len(chunk) // 4
            su = self.staging_info.uav_index
            self.run([("ew", [su, 0, 0, su, 0, 0, b.uav, (offset + s) // 4, 0, words, 1, 5], ((words + 255) // 256, 1, 1))])

    def read(self, b, offset, nbytes, dtype):
        out = np.empty(nbytes // np.dtype(dtype).itemsize, dtype)
        native.check(self.L.gd_readback(self.ctx, b.h, offset, nbytes, out.ctypes.data, TIMEOUT), "gd_readback")
        return out

    def close(self):
        for p in self.pipes.values():
            native.check(self.L.gd_release_pipeline(self.ctx, p, TIMEOUT), "gd_release_pipeline")
        for h in self.bufs:
            native.check(self.L.gd_release_buffer(self.ctx, h, TIMEOUT), "gd_release_buffer")
        native.check(self.L.gd_destroy(self.ctx, TIMEOUT), "gd_destroy")


def device_cus() -> int:
    """The device's CU count, as the engine reads it: hipDeviceGetAttribute with
    hipDeviceAttributeMultiprocessorCount (63 in hip_runtime_api.h)."""
    hip = C.CDLL("libamdhip64.so.7")  # the runtime the gd library links
    cu = C.c_int(0)
    assert hip.hipDeviceGetAttribute(C.byref(cu), 63, 0) == 0
    assert cu.value > 0
    return cu.value


@pytest.mark.gpu
@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_snippets_replay(oracle_mod, case):
    kind, L, x = make_case(case)
    n, E, U = x.shape[0], L.E, L.n_used
    path = PATH_PREFILL if kind.startswith("prefill") else PATH_DECODE
    ol = oracle_mod.OracleLayer(L)
    ref, tr = ol.forward(x, trace=True)
    logits = ol.router_f64(x)
    p = np.exp(logits - logits.max(axis=1, keepdims=True))
    s = -np.sort(-(p / p.sum(axis=1, keepdims=True)), axis=1)
    sep = (s[:, U - 1] - s[:, U]) > 1e-5 * s[:, U - 1]

    eng = Engine(max_tok=max(8, 16 * n) if path == PATH_PREFILL else 8)
    try:
        eng.add_layer(L)
        want = eng.forward(0, x, path)
        want_ids, want_w = eng.last_routes(n)
    finally:
        eng.close()

    dev = Device()
    try:
        ns = names(L, n, device_cus(), dev.buffer)
        calls = [evaluate(c, ns) for c in sequence(kind, ns)]
        print(f"{kind} E={E} F={L.F} experts={L.n_expert} top-{U} n={n} SF={L.SF}: "
              + ", ".join(f"{k}{list(g)}" for k, _, g in calls), flush=True)
        dev.write(ns.x, X_OFF * 4, x.tobytes())
        dev.run(calls)
        out = dev.read(ns.out, OUT_OFF * 4, n * E * 4, np.float32).reshape(n, E)
        ids = dev.read(ns.ids, 0, n * U * 4, np.uint32).reshape(n, U)
        w = dev.read(ns.weights, 0, n * U * 4, np.float32).reshape(n, U)
    finally:
        dev.close()

    np.testing.assert_array_equal(ids, want_ids)
    np.testing.assert_array_equal(w.view(np.uint32), want_w.view(np.uint32))
    np.testing.assert_array_equal(out.view(np.uint32), want.view(np.uint32))
    np.testing.assert_array_equal(ids[sep], tr["route_ids"][sep])
    np.testing.assert_allclose(w[sep], tr["route_w"][sep], rtol=2e-5, atol=1e-7)
    r, c = oracle_mod.rel_rms(ref, out), oracle_mod.cosine(ref, out)
    print(f"  replay == gm_forward bit for bit; rel_rms {r:.3e} cosine {c:.8f}; "
          f"{int((~sep).sum())} tokens near a routing tie", flush=True)
    assert r <= REL_RMS and c >= COSINE
