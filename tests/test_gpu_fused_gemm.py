"""GPU tests of the MFMA GEMM's fused SwiGLU epilogue.

The fused entry is held bit for bit against the unfused sequence it
replaces, run through the same library on the same inputs:

  wafer_hip_gemm_mfma_swiglu == two wafer_hip_gemm_mfma (narrow out, gate
      and up) followed by wafer_hip_silu_mul, in BF16 and in F16.

Both sides accumulate the same products in the same MFMA order, so the
narrowed products are identical and the region arithmetic is the same
function; any difference is a bug in the epilogue (a wrong column pairing, a
dropped rounding point, a tail store).  The unfused GEMM itself is held to
the formal lane in test_gpu_parity.py.  Shapes cover the 4-wave kernel's
256x224 and 256x256 tiles (the decoder layer's shape takes 256x224), the
8-wave kernel's full and ragged (m / feature tail) tiles, and one 16-feature
group.
"""
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    from vibe_compiler_amd import backend

    ctx = backend.Context(0)
    yield ctx
    ctx.close()


@pytest.fixture(scope="module")
def torch():
    import torch

    return torch


def _rnd(torch, gen, *shape, std=1.0, dt=None):
    return (torch.randn(*shape, generator=gen, device="cuda") * std).to(dt or torch.bfloat16)


def _same_bits(torch, a, b):
    return torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("fmt,m,k,f", [
    ("bf16", 1024, 4096, 14336),  # decoder layer gate/up (256x256 tiles)
    ("bf16", 256, 512, 512),
    ("bf16", 200, 256, 96),       # ragged m and a feature count that leaves a partial 256-column tile
    ("bf16", 64, 128, 32),        # two 16-feature groups
    ("bf16", 64, 128, 16),        # one 16-feature group
    ("bf16", 512, 1024, 1792),    # 256x224 tiles on the 4-wave kernel (n 3584)
    ("bf16", 256, 192, 128),      # 8-wave kernel, full tiles (K not a whole pair of 128-byte stages)
    ("f16", 16, 4096, 11008),     # the llama-2-7b-block FFN
    ("f16", 200, 256, 96),
    ("f16", 512, 1024, 1792),
])
def test_gemm_swiglu_bit_exact(hip, torch, fmt, m, k, f):
    from vibe_compiler_amd import backend as B

    fmt, dt = (B.BF16, torch.bfloat16) if fmt == "bf16" else (B.F16, torch.float16)
    gen = torch.Generator(device="cuda").manual_seed(20260803 + m + k + f)
    h = _rnd(torch, gen, m, k, dt=dt)
    wg, wu = _rnd(torch, gen, f, k, std=0.05, dt=dt), _rnd(torch, gen, f, k, std=0.05, dt=dt)
    gate = torch.empty(m, f, dtype=dt, device="cuda")
    up = torch.empty_like(gate)
    ref = torch.empty_like(gate)
    hip.gemm_mfma(h, wg, gate, m, k, f, in_fmt=fmt, out_fmt=fmt, rhs_t=True)
    hip.gemm_mfma(h, wu, up, m, k, f, in_fmt=fmt, out_fmt=fmt, rhs_t=True)
    hip.silu_mul(gate, up, ref, fmt=fmt)
    wgu = torch.empty(2 * f, k, dtype=dt, device="cuda")
    hip.interleave_gate_up(wg, wu, wgu)
    # canary past the output: a tail store beyond m*f would change it
    buf = torch.full((m * f + 64,), 1.5, dtype=dt, device="cuda")
    hip.gemm_mfma_swiglu(h, wgu, buf[: m * f].view(m, f), m, k, f, in_fmt=fmt)
    torch.cuda.synchronize()
    # the packing itself: 32-row groups of 16 gate rows then 16 up rows
    g4 = wgu.view(f // 16, 2, 16, k)
    assert torch.equal(g4[:, 0].reshape(f, k), wg) and torch.equal(g4[:, 1].reshape(f, k), wu)
    assert _same_bits(torch, buf[: m * f].view(m, f), ref)
    assert torch.all(buf[m * f:] == 1.5)


def test_fused_entries_reject_unsupported(hip, torch):
    from vibe_compiler_amd import backend as B

    t = torch.zeros(64 * 64, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(B.WaferHipError):
        hip.gemm_mfma_swiglu(t, t, t, 8, 64, 24)  # features not a multiple of 16
    r = t.view(torch.int16)  # raw 16-bit storage, so the library (not the wrapper) sees I16
    with pytest.raises(B.WaferHipError):
        hip.gemm_mfma_swiglu(r, r, r, 8, 64, 32, in_fmt=B.I16)  # bf16 / f16 only
