"""ORACLE — test infrastructure only.  Plain-PyTorch restatement of the
reference's checkpointed Llama decoder layer, used by tests/, by
``__graft_entry__.smoke()`` and by ``bench.py``'s cpu_baseline leg as the checker.
Nothing in the product (femtotron_amd/) imports it.

What it restates (transformers 5.15.0, the library the reference calls for the
layer arithmetic; femtotron itself has no arithmetic of its own on this path):
  rmsnorm           models/llama/modeling_llama.py:62-67
  rotate_half/rope  models/llama/modeling_llama.py:130-160
  mlp               models/llama/modeling_llama.py:174-176 (+ activations.py:93-103)
  attention         integrations/sdpa_attention.py:79-166 (causal, GQA via the
                    repeat_kv head mapping of modeling_llama.py:179-188, fp32 softmax)
  decoder_layer     models/llama/modeling_llama.py:295-325
  causal_lm_loss    femtotron/model/llama.py:91-111 (shifted fp32 cross-entropy)
  OracleLlama       femtotron/model/llama_partial_model.py:159-220 + llama.py:72-102

Every tensor op below runs in the input dtype, so bf16 inputs reproduce the
reference's op-by-op bf16 rounding and fp32 inputs its fp32 arithmetic.  The
functions are plain autograd code: gradients come from torch's autograd.

Pinning (tests/test_oracle.py): bit-for-bit / 1e-6 agreement with the Hugging
Face modules on CPU in fp32, agreement in bf16, the numpy fp64 closed forms in
oracle/closed_form.py (themselves pinned by finite differences and invariants),
and the golden fixtures written from the reference in tests/golden/.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    xf = x.to(torch.float32)
    var = xf.pow(2).mean(-1, keepdim=True)
    return w * (xf * torch.rsqrt(var + eps)).to(x.dtype)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def rope(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
    """q [B,nh,S,d], k [B,nkv,S,d], cos/sin [1|B,S,d]."""
    c, s = cos.unsqueeze(1), sin.unsqueeze(1)
    return (q * c) + (rotate_half(q) * s), (k * c) + (rotate_half(k) * s)


def repeat_kv(x: torch.Tensor, n_rep: int) -> torch.Tensor:
    """[B,nkv,S,d] -> [B,nkv*n_rep,S,d]; kv head j serves q heads j*n_rep .. j*n_rep+n_rep-1."""
    if n_rep == 1:
        return x
    B, nkv, S, d = x.shape
    return x[:, :, None].expand(B, nkv, n_rep, S, d).reshape(B, nkv * n_rep, S, d)


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float) -> torch.Tensor:
    """Causal softmax attention; scores and softmax in fp32 (fp64 for fp64
    inputs), output in q.dtype.
    Returns [B,S,nh*d] (the reference's transpose(1,2).reshape)."""
    B, nh, S, d = q.shape
    n_rep = nh // k.shape[1]
    acc = torch.float64 if q.dtype == torch.float64 else torch.float32
    kk = repeat_kv(k, n_rep).to(acc)
    vv = repeat_kv(v, n_rep).to(acc)
    scores = torch.matmul(q.to(acc), kk.transpose(-1, -2)) * scale
    mask = torch.ones(S, S, dtype=torch.bool, device=q.device).triu(1)
    scores = scores.masked_fill(mask, float("-inf"))
    probs = torch.softmax(scores, dim=-1)
    o = torch.matmul(probs, vv).to(q.dtype)
    return o.transpose(1, 2).reshape(B, S, nh * d)


def mlp(z: torch.Tensor, wg: torch.Tensor, wu: torch.Tensor, wd: torch.Tensor) -> torch.Tensor:
    return F.linear(F.silu(F.linear(z, wg)) * F.linear(z, wu), wd)


def decoder_layer(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, wts: dict,
                  n_heads: int, n_kv: int, head_dim: int, eps: float) -> torch.Tensor:
    """wts keys: wq wk wv wo wg wu wd w1 w2 (HF [out, in] layouts)."""
    B, S, _ = x.shape
    y = rmsnorm(x, wts["w1"], eps)
    q = F.linear(y, wts["wq"]).view(B, S, n_heads, head_dim).transpose(1, 2)
    k = F.linear(y, wts["wk"]).view(B, S, n_kv, head_dim).transpose(1, 2)
    v = F.linear(y, wts["wv"]).view(B, S, n_kv, head_dim).transpose(1, 2)
    q, k = rope(q, k, cos, sin)
    o = attention(q, k, v, head_dim ** -0.5)
    h = x + F.linear(o, wts["wo"])
    return h + mlp(rmsnorm(h, wts["w2"], eps), wts["wg"], wts["wu"], wts["wd"])


def rope_cos_sin(seq_len: int, head_dim: int, theta: float, dtype: torch.dtype,
                 inv_freq: torch.Tensor | None = None, device="cpu"):
    """cos/sin [1,S,d] as LlamaRotaryEmbedding.forward (modeling_llama.py:111-127):
    fp32 pos*inv_freq, cat(freqs,freqs), cos/sin, cast to dtype."""
    if inv_freq is None:
        inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    pos = torch.arange(seq_len, dtype=torch.float32, device=device)
    freqs = pos[:, None] * inv_freq.to(device=device, dtype=torch.float32)[None, :]
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos()[None].to(dtype), emb.sin()[None].to(dtype)


def causal_lm_loss(logits: torch.Tensor, labels: torch.Tensor) -> torch.Tensor:
    sl = logits[..., :-1, :].contiguous()
    tl = labels[..., 1:].contiguous()
    return F.cross_entropy(sl.float().view(-1, sl.size(-1)), tl.view(-1), ignore_index=-100)


LAYER_KEYS = ("wq", "wk", "wv", "wo", "wg", "wu", "wd", "w1", "w2")


def layer_weight_shapes(H: int, nh: int, nkv: int, hd: int, Fd: int) -> dict:
    """Parameter shapes in the reference's registration order within a layer
    (self_attn q,k,v,o; mlp gate,up,down; input_layernorm; post_attention_layernorm)."""
    return {"wq": (nh * hd, H), "wk": (nkv * hd, H), "wv": (nkv * hd, H), "wo": (H, nh * hd),
            "wg": (Fd, H), "wu": (Fd, H), "wd": (H, Fd), "w1": (H,), "w2": (H,)}


class OracleLlama:
    """Functional LlamaForTraining: embed -> layers -> norm -> lm_head -> loss.

    Parameters are drawn N(0, std) in the reference's registration order
    (embed, per layer q,k,v,o,gate,up,down,norm1,norm2, final norm, lm_head)
    from a CPU Generator(seed), exactly like init_llama_weights_ in the product."""

    def __init__(self, *, vocab: int, hidden: int, n_layers: int, n_heads: int, n_kv: int,
                 ffn: int, theta: float = 10000.0, eps: float = 1e-5, std: float = 0.02,
                 seed: int = 42, dtype: torch.dtype = torch.float32, device="cpu"):
        self.V, self.H, self.L, self.nh, self.nkv, self.F = vocab, hidden, n_layers, n_heads, n_kv, ffn
        self.hd = hidden // n_heads
        self.theta, self.eps, self.dtype, self.device = theta, eps, dtype, device
        gen = torch.Generator(device="cpu").manual_seed(seed)

        def draw(shape):
            return torch.empty(shape, dtype=torch.float32).normal_(0.0, std, generator=gen)

        self.embed = draw((vocab, hidden))
        self.layers = []
        for _ in range(n_layers):
            shapes = layer_weight_shapes(hidden, n_heads, n_kv, self.hd, ffn)
            self.layers.append({k: draw(shapes[k]) for k in LAYER_KEYS})
        self.norm = draw((hidden,))
        self.lm_head = draw((vocab, hidden))
        for t in self.params():
            t.data = t.data.to(device=device, dtype=dtype)
            t.requires_grad_(True)
        # inv_freq follows the model dtype cast, as in the reference (.bfloat16()
        # also casts buffers, femtotron/scripts/train.py:219).
        inv = 1.0 / (theta ** (torch.arange(0, self.hd, 2, dtype=torch.float32) / self.hd))
        self.inv_freq = inv.to(dtype).to(torch.float32)

    def params(self) -> list[torch.Tensor]:
        out = [self.embed]
        for lw in self.layers:
            out += [lw[k] for k in LAYER_KEYS]
        return out + [self.norm, self.lm_head]

    def named_params(self) -> list[tuple[str, torch.Tensor]]:
        hf = {"wq": "self_attn.q_proj.weight", "wk": "self_attn.k_proj.weight",
              "wv": "self_attn.v_proj.weight", "wo": "self_attn.o_proj.weight",
              "wg": "mlp.gate_proj.weight", "wu": "mlp.up_proj.weight",
              "wd": "mlp.down_proj.weight", "w1": "input_layernorm.weight",
              "w2": "post_attention_layernorm.weight"}
        out = [("model.embed_tokens.weight", self.embed)]
        for i, lw in enumerate(self.layers):
            out += [(f"model.layers.{i}.{hf[k]}", lw[k]) for k in LAYER_KEYS]
        return out + [("model.norm.weight", self.norm), ("lm_head.weight", self.lm_head)]

    def forward(self, ids: torch.Tensor, labels: torch.Tensor | None = None,
                checkpoint: bool = True, debug: bool = True):
        h = F.embedding(ids, self.embed)
        S = ids.shape[1]
        cos, sin = rope_cos_sin(S, self.hd, self.theta, self.dtype, self.inv_freq, h.device)
        for lw in self.layers:
            fn = lambda x, lw=lw: decoder_layer(x, cos, sin, lw, self.nh, self.nkv, self.hd, self.eps)
            if checkpoint:
                h = torch.utils.checkpoint.checkpoint(fn, h, use_reentrant=False, debug=debug)
            else:
                h = fn(h)
        h = rmsnorm(h, self.norm, self.eps)
        logits = F.linear(h, self.lm_head)
        loss = causal_lm_loss(logits, labels) if labels is not None else None
        return logits, loss


def finite_tolerance_ok(a: torch.Tensor, b: torch.Tensor, rtol: float, atol: float) -> bool:
    """Element-wise |a-b| <= atol + rtol*|b| (torch.allclose semantics)."""
    return bool(torch.all((a - b).abs() <= atol + rtol * b.abs()))


def rel_max_err(a: torch.Tensor, b: torch.Tensor) -> float:
    """max|a-b| / max|b| (the reference's tensor-level metric, test_pipeline_stage.py:82-128)."""
    den = b.abs().max().item()
    return (a - b).abs().max().item() / (den if den > 0 else 1.0) if math.isfinite(den) else math.inf
