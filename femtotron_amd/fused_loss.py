"""Fused lm_head + chunked cross-entropy: the loss head without full logits.

Reference loss head (femtotron/model/llama.py:91-111, femtotron/model/base.py:20-31):

    logits = lm_head(hidden)                                    # [B, S, V], model dtype
    loss = F.cross_entropy(logits[..., :-1, :].float().view(-1, V),
                           labels[..., 1:].view(-1), ignore_index=-100)

It materialises the logits in the model dtype and twice more in fp32 (the
``.float()`` copy and the log-softmax), ~0.38 MB per token at V = 32000, which
is the largest activation term of a checkpointed step.  Here the rows are
processed in chunks of at most ~256 MB of logits: per chunk one library GEMM
forms the logits, ``fh_ce_fwd_bwd`` computes the fp32 row losses and overwrites
the chunk with its gradient (softmax - onehot) / n_valid in the model dtype (the
rounding point of the reference's ``.float()`` backward), and two GEMMs turn it
into the chunk's input gradient (dlogits @ W, in the model dtype like the
reference) and its weight-gradient contribution (dlogits^T @ hidden,
accumulated across chunks in fp32 and rounded once).  Both gradients are
computed in the forward and scaled by the incoming gradient in the backward, so
nothing of size [tokens, V] outlives a chunk.

The next-token shift needs no copy: the labels are shifted instead
(``shift_labels``: position s takes label s+1, the last position of each
sequence is ignore_index), which pairs exactly the same (logits row, label)
pairs and counts the same number of valid labels as the reference.
"""
from __future__ import annotations

import torch

from . import ops

IGNORE_INDEX = -100
CHUNK_BYTES = 256 << 20  # logits bytes per chunk


def shift_labels(labels: torch.Tensor, ignore_index: int = IGNORE_INDEX) -> torch.Tensor:
    """[B, S] labels -> [B*S] next-token targets: out[b, s] = labels[b, s+1],
    ignore_index at s = S-1 (femtotron/model/llama.py:97-98 shifts the logits instead)."""
    out = torch.full_like(labels, ignore_index)
    out[:, :-1] = labels[:, 1:]
    return out.reshape(-1).contiguous()


def supported(hidden: torch.Tensor, weight: torch.Tensor) -> bool:
    """Whether the fused loss can run: HIP device, bf16/fp32, matching dtypes."""
    return (hidden.is_cuda and weight.is_cuda and hidden.device == weight.device
            and hidden.dtype in (torch.bfloat16, torch.float32) and weight.dtype == hidden.dtype
            and weight.dim() == 2 and weight.shape[1] == hidden.shape[-1]
            and weight.shape[0] % 8 == 0 and not torch.is_autocast_enabled())


class FusedLinearCrossEntropy(torch.autograd.Function):
    """loss = mean over non-ignored rows of CE(hidden2 @ weight^T, targets).
    Saved for backward: the input gradient [N, H] and the weight gradient."""

    @staticmethod
    def forward(ctx, hidden2, weight, targets):
        N, H = hidden2.shape
        V = weight.shape[0]
        dev = hidden2.device
        n_valid = (targets != IGNORE_INDEX).sum().to(torch.float32)
        inv_count = (1.0 / n_valid).reshape(1)  # inf when nothing is valid -> NaN loss, as torch
        need_dx, need_dw = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        dx = torch.empty_like(hidden2) if need_dx else None
        dw32 = torch.zeros(V, H, dtype=torch.float32, device=dev) if need_dw else None
        loss_sum = torch.zeros((), dtype=torch.float32, device=dev)
        chunk = max(256, (CHUNK_BYTES // (V * hidden2.element_size())) // 256 * 256)
        for r0 in range(0, N, chunk):
            r1 = min(N, r0 + chunk)
            x_c = hidden2[r0:r1]
            logits = torch.mm(x_c, weight.t())
            loss_rows = ops.ce_fwd_bwd_(logits, targets[r0:r1], inv_count, IGNORE_INDEX)
            loss_sum += loss_rows.sum()
            if need_dx:
                torch.mm(logits, weight, out=dx[r0:r1])
            if need_dw:
                if hidden2.dtype == torch.float32:
                    dw32.addmm_(logits.t(), x_c)
                else:
                    torch.addmm(dw32, logits.t(), x_c, out_dtype=torch.float32, out=dw32)
            del logits
        ctx.save_for_backward(dx, dw32.to(weight.dtype) if need_dw else None)
        return loss_sum * inv_count[0]

    @staticmethod
    def backward(ctx, grad):
        dx, dw = ctx.saved_tensors
        g = grad.to(torch.float32)

        def scaled(t):  # (t * g).to(t.dtype): fh_scale, one streaming pass
            if t is None:
                return None
            if t.numel() % 8 == 0 and t.data_ptr() % 16 == 0 and t.is_contiguous():
                return ops.scale(t, g)
            return (t * g).to(t.dtype)
        return scaled(dx), scaled(dw), None


def fused_causal_lm_loss(hidden: torch.Tensor, weight: torch.Tensor,
                         labels: torch.Tensor) -> torch.Tensor:
    """The reference's shifted next-token cross-entropy of ``hidden @ weight^T``
    (hidden [B, S, H], weight [V, H], labels [B, S], ignore_index -100)."""
    B, S, H = hidden.shape
    return FusedLinearCrossEntropy.apply(hidden.reshape(B * S, H).contiguous(), weight,
                                         shift_labels(labels))
