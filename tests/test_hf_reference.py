"""Pins the float32 decoder-layer reference the GPU tests use
(tests/decoder_reference.reference_layer) against the official Hugging Face
LlamaDecoderLayer, the layer the reference's llama-2-7b-block board case takes
its expected output from (test/Board/PyTorch/wafer_pytorch_board_cases.py:
817-866): MHA and GQA, non-unit norm weights, float32 on the CPU.  A dropped
RoPE term, a wrong mask side or a transposed projection moves the result far
beyond the bound."""
import pytest

torch = pytest.importorskip("torch")
pytest.importorskip("transformers")

from tests.decoder_reference import hf_layer, reference_layer  # noqa: E402


@pytest.mark.parametrize("Hq,Hkv", [(4, 4), (4, 2)])
def test_reference_layer_matches_hugging_face(Hq, Hkv):
    D, T, ffn = 128, 16, 1024
    Hd = Hq * D
    g = torch.Generator().manual_seed(Hq * 10 + Hkv)
    r = lambda *s: torch.randn(s, generator=g) * 0.02  # noqa: E731
    W = {"input_norm": 1 + 0.1 * torch.randn(Hd, generator=g), "post_norm": 1 + 0.1 * torch.randn(Hd, generator=g),
         "wqkv": r((Hq + 2 * Hkv) * D, Hd), "wo": r(Hd, Hd), "wgate": r(ffn, Hd), "wup": r(ffn, Hd),
         "wdown": r(Hd, ffn)}
    x = torch.randn(T, Hd, generator=g) * 0.125
    ref = reference_layer(torch, x, W, 1e-5, 1e4, Hq, Hkv, D)
    hf = hf_layer(torch, x, W, 1e-5, 1e4, Hq, Hkv, D, ffn, torch.float32)
    assert (ref - hf).abs().max().item() <= 1e-5
    # the update alone (the residual stream would hide a wrong attention)
    d_ref, d_hf = ref - x, hf - x
    assert ((d_ref - d_hf).norm() / d_hf.norm()).item() <= 1e-4
