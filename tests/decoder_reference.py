"""Float32 evaluations of the Llama decoder layer used as references by the
decoder-layer tests.

reference_layer is the math of the reference's CPU decoder-block reference
(test/Tools/Inputs/wafer_pytorch_xla_capture.py:1183-1260) in plain torch
float32.  hf_layer runs the official Hugging Face LlamaDecoderLayer, which the
reference's llama-2-7b-block board case builds its expected output from
(test/Board/PyTorch/wafer_pytorch_board_cases.py:817-866 through
test/Tools/Inputs/wafer_pytorch_xla_capture.py:993-1100: the layer in the
case's dtype, eval mode, on the CPU, causal over the fixture's static
sequence); test_hf_reference pins the first against the second.
"""
import math


def reference_layer(torch, x, W, eps, theta, Hq, Hkv, D):
    """float32 evaluation of the decoder layer on the same bf16 weights."""
    f = lambda t: t.float()
    T, Hd = x.shape
    xf = f(x)

    def rms(v, w):
        return v * torch.rsqrt((v * v).mean(-1, keepdim=True) + eps) * f(w)

    def rope(t):  # t [H, T, D]
        inv = 1.0 / (theta ** (torch.arange(0, D, 2, device=t.device, dtype=torch.float32) / D))
        ang = torch.arange(T, device=t.device, dtype=torch.float32)[:, None] * inv[None, :]
        emb = torch.cat([ang, ang], -1)
        rot = torch.cat([-t[..., D // 2:], t[..., :D // 2]], -1)
        return t * emb.cos() + rot * emb.sin()

    h = rms(xf, W["input_norm"])
    qkv = h @ f(W["wqkv"]).t()
    q = qkv[:, :Hq * D].reshape(T, Hq, D).permute(1, 0, 2)
    k = qkv[:, Hq * D:(Hq + Hkv) * D].reshape(T, Hkv, D).permute(1, 0, 2)
    v = qkv[:, (Hq + Hkv) * D:].reshape(T, Hkv, D).permute(1, 0, 2)
    q, k = rope(q), rope(k)
    g = Hq // Hkv
    k = k.repeat_interleave(g, 0).contiguous()
    v = v.repeat_interleave(g, 0).contiguous()
    s = torch.matmul(q.contiguous(), k.transpose(1, 2).contiguous()) / math.sqrt(D)
    s = s.masked_fill(torch.triu(torch.ones(T, T, dtype=torch.bool, device=x.device), 1), float("-inf"))
    o = torch.matmul(torch.softmax(s, -1), v)
    a = o.permute(1, 0, 2).reshape(T, Hq * D)
    x1 = xf + a @ f(W["wo"]).t()
    h2 = rms(x1, W["post_norm"])
    act = torch.nn.functional.silu(h2 @ f(W["wgate"]).t()) * (h2 @ f(W["wup"]).t())
    return x1 + act @ f(W["wdown"]).t()


def hf_layer(torch, x, W, eps, theta, Hq, Hkv, D, ffn, dtype):
    """The Hugging Face LlamaDecoderLayer on the CPU in `dtype` with the
    weights W (the DecoderLayer layout: wqkv rows q, k, v) and input x [T,
    hidden]; returns the [T, hidden] output in `dtype`."""
    from transformers import LlamaConfig
    from transformers.models.llama.modeling_llama import LlamaDecoderLayer, LlamaRotaryEmbedding

    T, Hd = x.shape
    cfg = LlamaConfig(hidden_size=Hd, intermediate_size=ffn, num_attention_heads=Hq, num_key_value_heads=Hkv,
                      head_dim=D, rms_norm_eps=eps, rope_theta=theta, max_position_embeddings=max(4096, T),
                      attention_bias=False, mlp_bias=False, hidden_act="silu")
    cfg._attn_implementation = "sdpa"  # causal when no mask is given
    layer = LlamaDecoderLayer(cfg, layer_idx=0).to(dtype).eval()
    c = lambda t: t.detach().to("cpu", dtype)  # noqa: E731
    wqkv = c(W["wqkv"])
    layer.load_state_dict({
        "self_attn.q_proj.weight": wqkv[:Hq * D], "self_attn.k_proj.weight": wqkv[Hq * D:(Hq + Hkv) * D],
        "self_attn.v_proj.weight": wqkv[(Hq + Hkv) * D:], "self_attn.o_proj.weight": c(W["wo"]),
        "mlp.gate_proj.weight": c(W["wgate"]), "mlp.up_proj.weight": c(W["wup"]),
        "mlp.down_proj.weight": c(W["wdown"]), "input_layernorm.weight": c(W["input_norm"]),
        "post_attention_layernorm.weight": c(W["post_norm"])})
    xc = c(x)[None]
    pos = torch.arange(T)[None]
    with torch.no_grad():
        pe = LlamaRotaryEmbedding(cfg)(xc, pos)
        out = layer(xc, attention_mask=None, position_ids=pos, position_embeddings=pe)
    out = out[0] if isinstance(out, tuple) else out
    return out.reshape(T, Hd)
