"""Graph replay of the entries the bench times: each call is captured into a
HIP graph on a side stream (as bench.py's timed region does), then the graph
is replayed three times with eager work between the replays (the output
cleared by a fill kernel, an eager call of the same entry on other inputs),
and every replay's output must be bit-identical to the eager run's."""

import math

import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def say(*a):
    print("[gpu-case]", *a, flush=True)


@pytest.fixture(scope="module")
def hip():
    from vibe_compiler_amd import backend

    ctx = backend.Context(0)
    yield ctx
    ctx.close()


@pytest.fixture(scope="module")
def B():
    from vibe_compiler_amd import backend

    return backend


def bits(t):
    return t.view(torch.int16) if t.element_size() == 2 else t.view(torch.int32)


def replay_matches_eager(call, out, other_call):
    """call() writes `out`; other_call() is the same entry on other inputs
    and outputs (eager work between replays)."""
    call()
    torch.cuda.synchronize()
    ref = out.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            call()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for r in range(3):
        out.zero_()
        other_call()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(bits(out), bits(ref)), f"replay {r} differs from the eager run"
    del graph


def rnd(shape, gen, dtype=torch.bfloat16):
    return torch.randn(shape, generator=gen, device="cuda").to(dtype)


def test_fa_prefill_graph_replay(hip):
    """The headline workload: [1,16,2048,128] bf16 causal."""
    say("graph replay: fa prefill")
    gen = torch.Generator(device="cuda").manual_seed(11)
    shape = (1, 16, 2048, 128)
    q, k, v = (rnd(shape, gen) for _ in range(3))
    q2, k2, v2 = (rnd(shape, gen) for _ in range(3))
    o, o2 = torch.empty(shape, dtype=torch.bfloat16, device="cuda"), torch.empty(shape, dtype=torch.bfloat16,
                                                                                   device="cuda")
    s = 1.0 / math.sqrt(128)
    replay_matches_eager(lambda: hip.attention_prefill(q, k, v, o, s, causal=True), o,
                         lambda: hip.attention_prefill(q2, k2, v2, o2, s, causal=True))


def test_fd_decode_graph_replay(hip):
    """FD decode over 16 chunks (chunk states in the context's workspace,
    sized by the eager call before the capture)."""
    say("graph replay: fd decode")
    gen = torch.Generator(device="cuda").manual_seed(12)
    q = rnd((8, 32, 1, 128), gen)
    kc, vc = rnd((8, 8, 4096, 128), gen), rnd((8, 8, 4096, 128), gen)
    q2 = rnd((8, 32, 1, 128), gen)
    o, o2 = torch.empty_like(q), torch.empty_like(q)
    s = 1.0 / math.sqrt(128)
    replay_matches_eager(lambda: hip.attention_decode(q, kc, vc, o, s, chunks=16), o,
                         lambda: hip.attention_decode(q2, kc, vc, o2, s, chunks=16, kv_len=3000))


def test_i8_gemm_kn_graph_replay(hip):
    """int8 GEMM with a [K,N] rhs read in place (no workspace)."""
    say("graph replay: i8 gemm [K,N]")
    gen = torch.Generator(device="cuda").manual_seed(13)
    m, k, n = 3072, 512, 4096
    a = torch.randint(-128, 128, (m, k), device="cuda", generator=gen, dtype=torch.int8)
    b = torch.randint(-128, 128, (k, n), device="cuda", generator=gen, dtype=torch.int8)
    sc = torch.rand(n, device="cuda", generator=gen) * 0.01
    a2 = torch.randint(-128, 128, (m, k), device="cuda", generator=gen, dtype=torch.int8)
    y, y2 = (torch.empty((m, n), dtype=torch.int16, device="cuda") for _ in range(2))
    replay_matches_eager(lambda: hip.gemm_i8(a, b, sc, y, m, k, n), y,
                         lambda: hip.gemm_i8(a2, b, sc, y2, m, k, n))


def test_mfma_gemm_split_k_graph_replay(hip, B):
    """bf16 MFMA GEMM on the split-K schedule: f32 partial tiles in the
    context's area (grown by the eager call), then the fold launch."""
    say("graph replay: mfma gemm split-k")
    gen = torch.Generator(device="cuda").manual_seed(14)
    m, k, n = 256, 8192, 1024
    a, a2 = rnd((m, k), gen), rnd((m, k), gen)
    bt = rnd((n, k), gen)
    y, y2 = (torch.empty((m, n), dtype=torch.float32, device="cuda") for _ in range(2))
    replay_matches_eager(lambda: hip.gemm_mfma(a, bt, y, m, k, n, in_fmt=B.BF16, out_fmt=B.F32, rhs_t=True), y,
                         lambda: hip.gemm_mfma(a2, bt, y2, m, k, n, in_fmt=B.BF16, out_fmt=B.F32, rhs_t=True))


def test_decoder_layer_graph_replay(hip):
    """The decoder layer forward (config 4: 8 backend calls, 9 kernels,
    split-K partials and the layer's intermediates reused across calls)."""
    say("graph replay: decoder layer")
    from vibe_compiler_amd import decoder_layer as DL

    gen = torch.Generator(device="cuda").manual_seed(15)
    W = DL.random_weights(torch, gen)
    x = torch.randn((1024, 4096), device="cuda", generator=gen).to(torch.bfloat16)
    x2 = torch.randn((1024, 4096), device="cuda", generator=gen).to(torch.bfloat16)
    y, y2 = torch.empty_like(x), torch.empty_like(x)
    layer = DL.DecoderLayer(hip, W, 1024)
    replay_matches_eager(lambda: layer.forward(x, y), y, lambda: layer.forward(x2, y2))


def test_graph_survives_workspace_growth(B):
    """A graph captured while the context's split-K partial area was small
    still replays correctly after a larger eager call on the same context
    grows the area: the outgrown buffer is kept until the context is
    destroyed, so the graph's partial tiles never land in memory handed out
    since (a torch tensor allocated after the growth keeps its contents)."""
    say("graph replay across workspace growth")
    hip = B.Context(0)
    gen = torch.Generator(device="cuda").manual_seed(16)
    k, n = 8192, 1024
    small_m, big_m = 256, 1024   # 4 and 16 MiB of f32 partials (4 splits)
    a = rnd((small_m, k), gen)
    bt = rnd((n, k), gen)
    y = torch.empty((small_m, n), dtype=torch.float32, device="cuda")
    call = lambda: hip.gemm_mfma(a, bt, y, small_m, k, n, in_fmt=B.BF16, out_fmt=B.F32, rhs_t=True)  # noqa: E731
    call()
    torch.cuda.synchronize()
    ref = y.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            call()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    # the larger eager call grows the partial area
    a_big = rnd((big_m, k), gen)
    y_big = torch.empty((big_m, n), dtype=torch.float32, device="cuda")
    hip.gemm_mfma(a_big, bt, y_big, big_m, k, n, in_fmt=B.BF16, out_fmt=B.F32, rhs_t=True)
    torch.cuda.synchronize()
    canary = torch.full((8 << 20,), 3.0, dtype=torch.float32, device="cuda")  # 32 MiB allocated after the growth
    for r in range(3):
        y.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, ref), f"replay {r} differs from the eager run"
        assert bool(torch.all(canary == 3.0)), f"replay {r} wrote into memory allocated after the growth"
    # the grown area serves the large shape as before
    y_big2 = torch.empty_like(y_big)
    hip.gemm_mfma(a_big, bt, y_big2, big_m, k, n, in_fmt=B.BF16, out_fmt=B.F32, rhs_t=True)
    torch.cuda.synchronize()
    assert torch.equal(y_big, y_big2)
    del graph
    hip.close()
