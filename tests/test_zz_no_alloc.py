"""The no-allocation FD decode entry (wafer_hip_attention_decode_noalloc),
called through the C ABI:
same arguments and kernels as wafer_hip_attention_decode, but the chunk-grid
path keeps its chunk states in the library's static device scratch instead
of the context workspace.  Its output is checked against the allocating
entry's (the same kernels in the same order, so bit-identical, which is
within the attention gate) on two calls in a row, the second smaller, for
the chunk-grid path (small batches, and GQA groups of 8) and for the group
path; a request whose chunk states exceed the scratch maximum fails before
any launch."""
import ctypes
import math

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

SCRATCH_STATES = 8192


def _noalloc(L):
    f = L.wafer_hip_attention_decode_noalloc
    f.restype = ctypes.c_int
    vp, u32 = ctypes.c_void_p, ctypes.c_uint32
    f.argtypes = [vp, u32, vp, vp, vp, vp, u32, u32, u32, u32, u32, u32, ctypes.c_float, u32]
    return f


def _case(B, Hq, Hkv, cap, kv_len, seed):
    gen = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn((B, Hq, 1, 128), device="cuda", generator=gen).to(torch.bfloat16)
    k = torch.randn((B, Hkv, cap, 128), device="cuda", generator=gen).to(torch.bfloat16)
    v = torch.randn((B, Hkv, cap, 128), device="cuda", generator=gen).to(torch.bfloat16)
    return q, k, v


def test_noalloc_decode_captured_as_first_call():
    """On a fresh context, the chunk-grid no-allocation call is captured into
    a HIP graph as the context's first call; the graph is replayed three
    times (output cleared between replays) and each replay is bit-identical
    to the allocating entry run eagerly on another context."""
    from vibe_compiler_amd import backend

    L = backend.load()
    B, Hq, Hkv, cap, kv_len, chunks = 2, 8, 2, 4096, 3000, 16
    print(f"[gpu-case] noalloc decode captured first: B={B} Hq={Hq} Hkv={Hkv} kv_len={kv_len}", flush=True)
    q, k, v = _case(B, Hq, Hkv, cap, kv_len, 31)
    scale = 1.0 / math.sqrt(128)
    o = torch.full((B, Hq, 1, 128), 7.0, dtype=torch.bfloat16, device="cuda")
    hip = backend.Context(0)
    f = _noalloc(L)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    status = []
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            status.append(f(hip._bind(), backend.BF16, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), B,
                            Hq, Hkv, kv_len, cap, 128, scale, chunks))
    torch.cuda.current_stream().wait_stream(side)
    assert status == [0], L.wafer_hip_last_error()
    ref_ctx = backend.Context(0)
    o_ref = torch.zeros_like(o)
    ref_ctx.attention_decode(q, k, v, o_ref, scale, chunks=chunks, kv_len=kv_len)
    torch.cuda.synchronize()
    for r in range(3):
        o.fill_(7.0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(o.view(torch.int16), o_ref.view(torch.int16)), f"replay {r}"
    del graph
    ref_ctx.close()
    hip.close()


@pytest.mark.parametrize("first,second", [
    ((2, 8, 2, 4096, 4000, 16), (1, 4, 1, 1024, 777, 8)),     # chunk grid, then a smaller one
    ((3, 32, 4, 2048, 2048, 16), (2, 16, 2, 512, 300, 4)),    # GQA 8 (chunk grid), then smaller
    ((64, 32, 8, 1024, 1000, 16), (48, 32, 8, 512, 512, 16)),  # the group path (no scratch)
])
def test_noalloc_decode_matches_allocating_entry(first, second):
    from vibe_compiler_amd import backend

    L = backend.load()
    hip = backend.Context(0)
    f = _noalloc(L)
    for i, (B, Hq, Hkv, cap, kv_len, chunks) in enumerate((first, second)):
        print(f"[gpu-case] noalloc decode call {i}: B={B} Hq={Hq} Hkv={Hkv} cap={cap} kv_len={kv_len} "
              f"chunks={chunks}", flush=True)
        q, k, v = _case(B, Hq, Hkv, cap, kv_len, 100 + i)
        scale = 1.0 / math.sqrt(128)
        o_ref = torch.zeros((B, Hq, 1, 128), dtype=torch.bfloat16, device="cuda")
        hip.attention_decode(q, k, v, o_ref, scale, chunks=chunks, kv_len=kv_len)
        o = torch.full((B, Hq, 1, 128), 7.0, dtype=torch.bfloat16, device="cuda")
        st = f(hip._bind(), backend.BF16, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), B, Hq, Hkv,
               kv_len, cap, 128, scale, chunks)
        assert st == 0, L.wafer_hip_last_error()
        torch.cuda.synchronize()
        assert torch.equal(o.view(torch.int16), o_ref.view(torch.int16))
        # and against a float32 evaluation, to the attention gate
        kf = k[:, :, :kv_len].float().repeat_interleave(Hq // Hkv, 1)
        vf = v[:, :, :kv_len].float().repeat_interleave(Hq // Hkv, 1)
        s = (q.float() @ kf.transpose(-1, -2).contiguous()) * scale
        ref = torch.softmax(s, -1) @ vf
        g, r = o.float().flatten().double(), ref.flatten().double()
        cos = float(g @ r / (g.norm() * r.norm()))
        rel = float((g - r).norm() / r.norm())
        assert cos >= 0.9999 and rel <= 0.01, (cos, rel)
    hip.close()


def test_noalloc_decode_rejects_beyond_scratch():
    from vibe_compiler_amd import backend

    L = backend.load()
    hip = backend.Context(0)
    f = _noalloc(L)
    # 2 x 32 x 256 = 16384 chunk states on the chunk-grid path (> 8192)
    B, Hq, Hkv, cap, chunks = 2, 32, 4, 1024, 256
    q, k, v = _case(B, Hq, Hkv, cap, cap, 7)
    o = torch.full((B, Hq, 1, 128), 7.0, dtype=torch.bfloat16, device="cuda")
    st = f(hip._bind(), backend.BF16, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), B, Hq, Hkv, cap, cap,
           128, 0.088, chunks)
    assert st == -3
    assert b"scratch maximum" in L.wafer_hip_last_error()
    torch.cuda.synchronize()
    assert bool(torch.all(o == 7.0))  # nothing launched
    hip.close()
