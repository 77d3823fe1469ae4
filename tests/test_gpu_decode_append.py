"""GPU parity for decode with the functional KV-cache append
(wafer_hip_attention_decode_append): the reference's decode board cases
(test/Board/PyTorch/wafer_pytorch_board_cases.py:1098-1135
attention-causal-decode-two-tokens, :1138-1360 attention-decode-kv-cache with
its continuation step) and the FD classification they exercise
(lib/Wafer/Transforms/Linalg/AttentionMatching.cpp:1385-1437).

Checks per step:
  * the updated caches: rows before past_len bit-identical to the caches given
    (the cases' validate_actual_outputs), the appended rows bit-identical to
    the new K / V, rows past the append untouched;
  * the attention output against the CPU oracle (oracle_attention_decode for
    one token at head_dim 128, oracle_attention_prefill_ex with the
    lower-right causal diagonal otherwise) under the reference's attention
    policy plus elementwise rtol 0.006 / atol 0.008 (tests/similarity.py), and
    against float64 softmax attention;
  * the continuation: step 2 consumes step 1's updated caches in place.
"""
import math
import sys

import numpy as np
import pytest

from tests.similarity import attention_gate

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

F16, BF16 = 2, 3


def say(*a):
    print("[gpu-append]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def hip():
    from vibe_compiler_amd import backend

    ctx = backend.Context(0)
    yield ctx
    ctx.close()


def u16(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint16).view(np.int16)).cuda()


def back(t):
    torch.cuda.synchronize()
    return t.cpu().numpy().view(np.uint16)


def store(oracle, fmt, x):
    x = np.asarray(x, np.float32)
    if fmt == BF16:
        return oracle.f32_to_bf16(x).reshape(x.shape)
    return x.astype(np.float16).view(np.uint16)


def tof(oracle, fmt, a):
    return oracle.to_float(fmt, a).reshape(a.shape)


def sdpa64(oracle, fmt, q, k, v, past):
    """float64 softmax attention, query i seeing keys j <= past + i (GQA by head groups)."""
    qf, kf, vf = (tof(oracle, fmt, t).astype(np.float64) for t in (q, k, v))
    g = qf.shape[1] // kf.shape[1]
    kf = np.repeat(kf, g, axis=1)
    vf = np.repeat(vf, g, axis=1)
    s = qf @ np.swapaxes(kf, -1, -2) / math.sqrt(qf.shape[-1])
    T, L = s.shape[-2], s.shape[-1]
    s = np.where(np.arange(L)[None, :] <= past + np.arange(T)[:, None], s, -np.inf)
    s = s - s.max(-1, keepdims=True)
    p = np.exp(s)
    return (p / p.sum(-1, keepdims=True)) @ vf


def decode_step(hip, oracle, fmt, q, kn, vn, kc, vc, past, chunks=16):
    """Run one append step on the device caches kc / vc (torch int16) and
    check the caches and the output; returns the output bits."""
    Bn, Hq, T, D = q.shape
    cap = kc.shape[2]
    before_k, before_v = back(kc).copy(), back(vc).copy()
    o = torch.full((Bn, Hq, T, D), 0x7E00, dtype=torch.int16, device="cuda")
    hip.attention_decode_append(u16(q), u16(kn), u16(vn), kc, vc, o, 1.0 / math.sqrt(D), past, chunks=chunks, fmt=fmt)
    got = back(o)
    after_k, after_v = back(kc), back(vc)
    for name, before, after, new in (("K", before_k, after_k, kn), ("V", before_v, after_v, vn)):
        assert np.array_equal(after[:, :, :past], before[:, :, :past]), f"{name} prefix changed"
        assert np.array_equal(after[:, :, past:past + T], new), f"{name} appended rows differ"
        assert np.array_equal(after[:, :, past + T:], before[:, :, past + T:]), f"{name} rows past the append changed"
    L = past + T
    scale = 1.0 / math.sqrt(D)
    if T == 1 and D == 128:
        ref = oracle.attention_decode(q, after_k, after_v, scale, chunks=chunks, kv_len=L, block_k=64, fmt=fmt)
    else:
        ref = oracle.attention_prefill_ex(q, after_k, after_v, scale, kv_len=L, causal=True, diagonal=past, fmt=fmt)
    attention_gate(tof(oracle, fmt, got), tof(oracle, fmt, ref), what=f"append step past={past} vs oracle")
    attention_gate(tof(oracle, fmt, got), sdpa64(oracle, fmt, q, after_k[:, :, :L], after_v[:, :, :L], past),
                   what=f"append step past={past} vs float64")
    return got


@pytest.mark.parametrize("fmt", [F16, BF16], ids=["f16", "bf16"])
@pytest.mark.parametrize("cap", [1026, 1040])
def test_causal_decode_two_tokens(hip, oracle, fmt, cap):
    """attention-causal-decode-two-tokens: q / new K / new V [1,1,2,64],
    past caches [1,1,1024,64], every input scaled by 0.125; SDPA with
    causal_lower_right(2, 1026); outputs (attention, keys, values)."""
    say("two tokens", fmt, cap)
    rng = np.random.default_rng(1098 + fmt + cap)
    mk = lambda n: store(oracle, fmt, rng.standard_normal((1, 1, n, 64)) * 0.125)
    q, kn, vn = mk(2), mk(2), mk(2)
    kc = u16(np.concatenate([mk(1024), mk(cap - 1024)], axis=2))
    vc = u16(np.concatenate([mk(1024), mk(cap - 1024)], axis=2))
    decode_step(hip, oracle, fmt, q, kn, vn, kc, vc, past=1024)


@pytest.mark.parametrize("fmt", [F16, BF16], ids=["f16", "bf16"])
@pytest.mark.parametrize("past0,cap", [(1023, 1040), (4094, 4096)], ids=["kv-cache", "kv-cache-long-4096"])
def test_decode_kv_cache_two_steps(hip, oracle, fmt, past0, cap):
    """attention-decode-kv-cache at the Llama-2-7B layer shapes (32 heads MHA,
    head_dim 128, past 1023): step 1 appends one token and runs FD over 1024
    keys; the continuation consumes step 1's updated caches (past 1024 -> 1025
    keys).  attention-decode-kv-cache-long-4096 (:1528-1530) is the same two
    steps from past 4094, ending with the cache full at 4096
    (max_position_embeddings).  The case's projections and RoPE stay outside
    the attention command; q and the new K / V are drawn directly."""
    say("kv cache two steps", fmt, past0)
    rng = np.random.default_rng(1138 + fmt + past0)
    Hq, D = 32, 128
    kc = u16(store(oracle, fmt, rng.standard_normal((1, Hq, cap, D)) * 0.125))
    vc = u16(store(oracle, fmt, rng.standard_normal((1, Hq, cap, D))))
    past = past0
    step1_k = None
    for step in range(2):
        q = store(oracle, fmt, rng.standard_normal((1, Hq, 1, D)) * 0.125)
        kn = store(oracle, fmt, rng.standard_normal((1, Hq, 1, D)) * 0.125)
        vn = store(oracle, fmt, rng.standard_normal((1, Hq, 1, D)))
        decode_step(hip, oracle, fmt, q, kn, vn, kc, vc, past=past)
        if step == 0:
            step1_k = back(kc)[:, :, :past + 1].copy()
        else:
            # the continuation kept step 1's updated cache as its prefix
            assert np.array_equal(back(kc)[:, :, :past], step1_k)
        past += 1


@pytest.mark.parametrize("fmt", [F16, BF16], ids=["f16", "bf16"])
@pytest.mark.parametrize("Bn,Hq,Hkv,T,D,past,cap,chunks", [
    (2, 32, 8, 1, 128, 4095, 4100, 16),   # GQA 4, FD chunk grid
    (64, 8, 2, 1, 128, 700, 701, 8),      # FD group path, cache full after the append
    (1, 8, 2, 3, 128, 500, 512, 16),      # three new tokens: masked prefill path
    (2, 4, 4, 5, 64, 77, 90, 16),
    (1, 2, 1, 2, 16, 33, 40, 16),         # head_dim 16: the one-thread-per-row lane
])
def test_decode_append_shapes(hip, oracle, fmt, Bn, Hq, Hkv, T, D, past, cap, chunks):
    say("append shapes", fmt, Bn, Hq, Hkv, T, D, past, cap, chunks)
    rng = np.random.default_rng(past + T + D + fmt)
    q = store(oracle, fmt, rng.standard_normal((Bn, Hq, T, D)) * 0.125)
    kn = store(oracle, fmt, rng.standard_normal((Bn, Hkv, T, D)) * 0.125)
    vn = store(oracle, fmt, rng.standard_normal((Bn, Hkv, T, D)))
    kc = u16(store(oracle, fmt, rng.standard_normal((Bn, Hkv, cap, D)) * 0.125))
    vc = u16(store(oracle, fmt, rng.standard_normal((Bn, Hkv, cap, D))))
    decode_step(hip, oracle, fmt, q, kn, vn, kc, vc, past=past, chunks=chunks)


def test_decode_append_rejects_overflow_without_writing(hip):
    """past_len + tokens beyond the capacity fails before any launch: the
    caches are left as they were."""
    from vibe_compiler_amd import backend as B

    kc = torch.arange(4 * 128, dtype=torch.int16, device="cuda").reshape(1, 1, 4, 128)
    vc = kc.clone()
    q = torch.zeros((1, 1, 2, 128), dtype=torch.int16, device="cuda")
    kn = torch.ones((1, 1, 2, 128), dtype=torch.int16, device="cuda")
    o = torch.zeros_like(q)
    L = B.load()
    st = L.wafer_hip_attention_decode_append(hip._bind(), BF16, B._p(q), B._p(kn), B._p(kn), B._p(kc), B._p(vc), B._p(o),
                                             1, 1, 1, 2, 3, 4, 128, 0.1, 16)
    assert st == -1
    assert b"exceeds kv_capacity" in L.wafer_hip_last_error()
    torch.cuda.synchronize()
    assert torch.equal(kc, vc) and int(kc[0, 0, 3, 127]) == 4 * 128 - 1
    with pytest.raises(ValueError):
        hip.attention_decode_append(q, kn, kn, kc, vc, o, 0.1, 3)
    assert L.wafer_hip_attention_decode_append(hip._bind(), BF16, B._p(q), B._p(kn), B._p(kn), B._p(kc), B._p(vc),
                                               B._p(o), 1, 1, 1, 2, 1, 4, 96, 0.1, 16) == -3
