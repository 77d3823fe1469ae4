"""CPU checks of the Python host binding's argument validation: every
wrapper compares each tensor's element width, floating dtype and size with
the format and shape it is called with, and raises ValueError before it
binds a stream or passes a pointer to the C ABI (which takes bare pointers
and cannot check extents: a short tensor would be written past its end on
the GPU).  A Context object is made without a device (its constructor is
skipped), so any call that got past the checks would fail on the missing
handle instead of raising ValueError."""
import pytest

torch = pytest.importorskip("torch")

from vibe_compiler_amd import backend as B  # noqa: E402


@pytest.fixture
def ctx():
    c = object.__new__(B.Context)
    c._h = None
    c._L = None
    c._torch = torch
    c.device = 0
    return c


def z(n, dt=torch.int16):
    return torch.zeros(n, dtype=dt)


CASES = [
    # (name, call) -- each call has exactly one bad operand
    ("gemm_mfma short dst", lambda c: c.gemm_mfma(z(64), z(64), z(63, torch.float32), 8, 8, 8)),
    ("gemm_mfma f16 tensor as bf16", lambda c: c.gemm_mfma(z(64, torch.float16), z(64), z(64, torch.float32), 8, 8, 8)),
    ("swiglu short rhs", lambda c: c.gemm_mfma_swiglu(z(64 * 32), z(64 * 63), z(32 * 32), 32, 64, 32)),
    ("gemm_i8 short a", lambda c: c.gemm_i8(z(100, torch.int8), z(64 * 128, torch.int8), z(128, torch.float32),
                                            z(128), 2, 64, 128)),
    ("gemm_i8 2-byte scale", lambda c: c.gemm_i8(z(64, torch.int8), z(64, torch.int8), z(1), z(1), 1, 64, 1)),
    ("gemm_i8 short acc", lambda c: c.gemm_i8(z(64, torch.int8), z(64, torch.int8), z(1, torch.float32), z(1), 1, 64,
                                              1, acc_out=z(0, torch.int32))),
    ("elementwise short in1", lambda c: c.elementwise("Add", B.BF16, z(16), z(16), in1=z(15))),
    ("elementwise missing in1", lambda c: c.elementwise("Mul", B.BF16, z(16), z(16))),
    ("elementwise f32 dst for bf16", lambda c: c.elementwise("Abs", B.BF16, z(16), z(16, torch.float32))),
    ("convert short dst", lambda c: c.convert(167, z(16, torch.float32), z(15))),
    ("reduce short dst", lambda c: c.reduce(B.REDUCE_SUM, 0, B.F32, [4, 8], z(32, torch.float32), z(3, torch.float32))),
    ("pack short logical", lambda c: c.pack(B.F32, B.TENSOR, [4, 8], z(31, torch.float32), z(32, torch.float32))),
    ("unpack short storage", lambda c: c.unpack(B.F32, B.TENSOR, [4, 8], z(31, torch.float32), z(32, torch.float32))),
    ("prefill short o", lambda c: c.attention_prefill(z(256).view(1, 1, 2, 128), z(256).view(1, 1, 2, 128),
                                                      z(256).view(1, 1, 2, 128), z(255), 0.1)),
    ("prefill v shape", lambda c: c.attention_prefill(z(256).view(1, 1, 2, 128), z(256).view(1, 1, 2, 128),
                                                      z(384).view(1, 1, 3, 128), z(256), 0.1)),
    ("prefill f16 q as bf16", lambda c: c.attention_prefill(z(256, torch.float16).view(1, 1, 2, 128),
                                                            z(256).view(1, 1, 2, 128), z(256).view(1, 1, 2, 128),
                                                            z(256), 0.1)),
    ("decode short o", lambda c: c.attention_decode(z(256).view(1, 2, 1, 128), z(512).view(1, 1, 4, 128),
                                                    z(512).view(1, 1, 4, 128), z(255), 0.1)),
    ("decode kv_len > cap", lambda c: c.attention_decode(z(256).view(1, 2, 1, 128), z(512).view(1, 1, 4, 128),
                                                         z(512).view(1, 1, 4, 128), z(256), 0.1, kv_len=5)),
    ("rmsnorm short w", lambda c: c.rmsnorm(z(64).view(2, 32), z(31), z(64), 1e-5)),
    ("rmsnorm short y", lambda c: c.rmsnorm(z(64).view(2, 32), z(32), z(63), 1e-5)),
    ("softmax short y", lambda c: c.softmax(z(64).view(2, 32), z(63))),
    ("silu_mul short up", lambda c: c.silu_mul(z(64), z(63), z(64))),
    ("gelu f32 y for bf16", lambda c: c.gelu_tanh(z(64), z(64, torch.float32))),
    ("rope short y", lambda c: c.rope(z(256).view(2, 1, 128), z(255), z(2, torch.int32), 1e4)),
    ("rope 2-byte positions", lambda c: c.rope(z(256).view(2, 1, 128), z(256), z(2), 1e4)),
    ("head_permute_rope 4-byte src for bf16", lambda c: c.head_permute_rope(z(256, torch.float32), z(256), 2, 1, 128,
                                                                            128, z(2, torch.int32), 1e4)),
    ("bias_add 2-byte bias", lambda c: c.bias_add(z(64, torch.float32).view(2, 32), z(32), z(64, torch.float32))),
    ("bias_add short y", lambda c: c.bias_add(z(64, torch.float32).view(2, 32), z(32, torch.float32),
                                              z(63, torch.float32))),
    ("mask_move 4-byte mask for f16", lambda c: c.mask_move(z(8), z(8, torch.float32), z(8), B.F16)),
    ("bit2fp short dst", lambda c: c.bit2fp(z(1, torch.uint8), z(7), B.BF16, 8)),
    ("first_nan short values", lambda c: c.first_nan(B.BF16, z(4), 5)),
]


@pytest.mark.parametrize("name,call", CASES, ids=[c[0] for c in CASES])
def test_wrapper_rejects_before_the_c_call(ctx, name, call):
    with pytest.raises(ValueError):
        call(ctx)


def test_valid_arguments_reach_the_binding(ctx):
    """The checks pass well-formed operands through: the call then fails on
    the device-less context, not with ValueError."""
    with pytest.raises(Exception) as e:
        ctx.silu_mul(z(64), z(64), z(64))
    assert not isinstance(e.value, ValueError)
