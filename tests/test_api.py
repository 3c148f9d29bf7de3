"""Host-side behaviour of the drop-in API (CPU; no GPU needed).

Mirrors what the reference's AC API promises (femtotron/training/
activation_ckpt.py, ckpt_policy.py, ckpt_config.py, scripts/presets.py) and the
C-ABI library's loadability: every symbol include/femtohip.h declares is
exported, and argument validation runs on the host before any launch.
"""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch
from torch import nn

from femtotron_amd import dispatch_counts, fused_checkpoint, reset_dispatch_counts
from femtotron_amd.training import (ALWAYS, NEVER, ActivationCheckpointWrapper, all_of, any_of,
                                    apply_activation_checkpointing, by_class, by_class_name,
                                    is_activation_checkpointed, not_of, policy_from_config,
                                    remove_activation_checkpointing)
from oracle import torch_llama as ot
from tests.helpers import CFG1, llama_config

ROOT = Path(__file__).resolve().parent.parent


class Block(nn.Module):
    def __init__(self):
        super().__init__()
        self.lin = nn.Linear(4, 4)

    def forward(self, x):
        return torch.relu(self.lin(x))


class Net(nn.Module):
    def __init__(self):
        super().__init__()
        self.blocks = nn.ModuleList([Block(), Block()])
        self.head = nn.Linear(4, 2)

    def forward(self, x):
        for b in self.blocks:
            x = b(x)
        return self.head(x)


def test_apply_counts_and_keeps_state_dict_keys():
    net = Net()
    keys = list(net.state_dict())
    params = list(net.parameters())
    assert apply_activation_checkpointing(net, by_class(Block)) == 2
    assert all(is_activation_checkpointed(b) for b in net.blocks)
    assert sorted(net.state_dict()) == sorted(keys)
    assert [id(p) for p in net.parameters()] == [id(p) for p in params]
    # load_state_dict with plain keys works through the wrapper
    net.load_state_dict({k: torch.zeros_like(v) for k, v in Net().state_dict().items()})
    assert torch.count_nonzero(net.blocks[0].inner_module.lin.weight) == 0
    # a policy selecting a module that contains a wrapper raises
    with pytest.raises(ValueError, match="nested"):
        apply_activation_checkpointing(net, by_class_name("ModuleList"))
    assert remove_activation_checkpointing(net) == 2
    assert remove_activation_checkpointing(net) == 0
    assert isinstance(net.blocks[0], Block)


def test_wrapper_forwards_debug_true_and_flags():
    seen = {}

    def fake_ckpt(fn, *args, **kw):
        seen.update(kw)
        return fn(*args)

    w = ActivationCheckpointWrapper(Block(), checkpoint_fn=fake_ckpt, use_reentrant=False,
                                    preserve_rng_state=True)
    w(torch.randn(3, 4))
    assert seen == {"use_reentrant": False, "preserve_rng_state": True, "debug": True}
    assert "use_reentrant=False" in repr(w)


def test_policies_and_config():
    b, n = Block(), Net()
    assert by_class(Block)(b) and not by_class(Block)(n)
    assert by_class_name("Net")(n)
    assert any_of(by_class(Block), by_class_name("Net"))(n)
    assert not all_of(by_class(Block), by_class_name("Net"))(b)
    assert not_of(by_class(Block))(n)
    assert NEVER(b) is False and ALWAYS(b) is True
    assert by_class(Block).__name__ == "by_class(Block)"
    for bad in (lambda: by_class(), lambda: by_class_name(), lambda: any_of(), lambda: all_of()):
        with pytest.raises(ValueError):
            bad()
    p = policy_from_config({"type": "any_of", "policies": [
        {"type": "by_class_name", "names": ["Block"]}, {"type": "not_of", "policy": {"type": "always"}}]})
    assert p(b) and not p(n)
    assert policy_from_config(None) is NEVER
    with pytest.raises(ValueError):
        policy_from_config({"type": "by_class_name", "names": "Block"})
    with pytest.raises(ValueError):
        policy_from_config({"type": "bogus"})


def test_presets():
    from transformers.models.llama.modeling_llama import LlamaDecoderLayer, LlamaMLP
    from femtotron_amd.scripts.presets import get_ac_policy, get_wrap_policy
    layer = LlamaDecoderLayer(llama_config(CFG1, layers=1), 0)
    assert get_ac_policy("llama_decoder_layer")(layer)
    assert get_wrap_policy("llama_decoder_layer")(layer)
    assert get_ac_policy("llama_mlp_and_norms")(layer.mlp)
    assert not get_ac_policy("llama_mlp_and_norms")(layer.self_attn)
    with pytest.raises(ValueError, match="Available"):
        get_ac_policy("nope")


def test_fused_checkpoint_on_cpu_is_the_stock_checkpoint():
    """CPU tensors are not the fused path's domain: results and gradients equal
    torch.utils.checkpoint exactly, and the call is counted as a fallback."""
    from transformers.models.llama.modeling_llama import LlamaDecoderLayer
    torch.manual_seed(0)
    layer = LlamaDecoderLayer(llama_config(CFG1, layers=1), 0)
    S = 16
    cos, sin = ot.rope_cos_sin(S, 32, 1e4, torch.float32)
    x = torch.randn(2, S, 256)
    outs = []
    for fn in (fused_checkpoint, torch.utils.checkpoint.checkpoint):
        layer.zero_grad()
        xi = x.clone().requires_grad_(True)
        reset_dispatch_counts()
        y = fn(layer, xi, use_reentrant=False, preserve_rng_state=True, debug=True,
               attention_mask=None, position_embeddings=(cos, sin), past_key_values=None,
               use_cache=False)
        y.sum().backward()
        outs.append((y.detach(), xi.grad, layer.self_attn.q_proj.weight.grad.clone()))
        if fn is fused_checkpoint:
            assert dispatch_counts() == {"fused": 0, "fallback": 1}
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    with pytest.raises(ValueError):
        fused_checkpoint(layer, x, use_reentrant=True, debug=True, position_embeddings=(cos, sin))


def test_dispatcher_recognises_layer_mlp_and_norm_only():
    """The fused path claims HF's decoder layer, MLP and RMSNorm (the modules the
    full and selective presets wrap) and nothing else; a subclass that overrides
    forward is not claimed.  On CPU tensors every call still falls back."""
    from transformers.models.llama import modeling_llama as hf
    from femtotron_amd.fused_checkpoint import _kind, _plan
    cfg = llama_config(CFG1, layers=1)
    layer = hf.LlamaDecoderLayer(cfg, 0)

    class CustomMLP(hf.LlamaMLP):
        def forward(self, x):
            return super().forward(x) * 2

    assert _kind(layer) == "layer"
    assert _kind(layer.mlp) == "mlp"
    assert _kind(layer.input_layernorm) == "norm"
    assert _kind(layer.self_attn) is None
    assert _kind(CustomMLP(cfg)) is None
    assert "not an unmodified" in _plan(CustomMLP(cfg), (torch.randn(1, 4, 256),), {})
    assert "HIP" in _plan(layer.mlp, (torch.randn(1, 4, 256),), {})
    x = torch.randn(1, 4, 256, requires_grad=True)
    reset_dispatch_counts()
    y = fused_checkpoint(layer.mlp, x, use_reentrant=False, debug=True)
    assert dispatch_counts() == {"fused": 0, "fallback": 1}
    assert torch.equal(y, layer.mlp(x))


# --------------------------------------------------------------- C ABI
def _declared_symbols() -> set[str]:
    text = (ROOT / "include" / "femtohip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(fh_[a-z0-9_]+)\s*\(", text))


def test_library_exports_every_declared_symbol():
    from femtotron_amd import _lib
    if not _lib.LIB_PATH.exists():
        pytest.skip("libfemtohip.so not built")
    declared = _declared_symbols()
    assert declared, "no declarations parsed"
    assert declared == set(_lib.SIGNATURES), declared ^ set(_lib.SIGNATURES)
    raw = ctypes.CDLL(str(_lib.LIB_PATH))
    for name in declared:
        assert hasattr(raw, name), name
    assert _lib.lib().fh_abi_version() == _lib.ABI_VERSION


def test_library_validates_arguments_on_host():
    """Invalid arguments are rejected before any HIP call (works without a GPU)."""
    from femtotron_amd import _lib
    if not _lib.LIB_PATH.exists():
        pytest.skip("libfemtohip.so not built")
    L = _lib.lib()
    assert L.fh_rmsnorm_fwd(7, None, None, None, None, 1, 64, 1e-5, None) == 1  # bad dtype
    assert b"dtype" in L.fh_last_error()
    assert L.fh_rmsnorm_fwd(0, None, None, None, None, 1, 12, 1e-5, None) == 1  # cols % 8
    assert L.fh_rope_fwd(0, None, 64, 4, 4, 2, 24, None, None, 0, None) == 1     # head_dim % 16
    assert L.fh_swiglu_fwd(0, None, None, 8, None, 8, 0, 8, None) == 0           # empty is a no-op
    assert L.fh_rmsnorm_bwd_workspace_size(0, 64) == 0
    assert L.fh_rmsnorm_bwd_workspace_size(16384, 2048) > 0
    # projection GEMM: op, k % 64 and alignment are checked before any launch
    assert L.fh_gemm_bf16(7, None, 64, None, 64, None, 64, None, 0, 64, 64, 64, None, None) == 1
    assert b"op" in L.fh_last_error()
    assert L.fh_gemm_bf16(_lib.FH_GEMM_NN, None, 96, None, 64, None, 64, None, 0, 64, 64, 96,
                          None, None) == 1
    assert b"multiple of 64" in L.fh_last_error()
    assert L.fh_gemm_bf16(_lib.FH_GEMM_NT, None, 64, None, 64, None, 64, None, 0, 64, 64, 64,
                          None, None) == 1  # null pointers
    # a 512 x 512 weight gradient over 16384 tokens is split into k slices
    assert L.fh_gemm_bf16_workspace_size(_lib.FH_GEMM_TN, 512, 512, 16384) > 0
    assert L.fh_gemm_bf16_workspace_size(_lib.FH_GEMM_NT, 16384, 2048, 2048) == 0
    assert L.fh_gemm_bf16_workspace_size(_lib.FH_GEMM_NT, 64, 64, 96) == 0


def test_linear_weight_accepts_tensor_parallel_wrappers_at_world_size_1():
    """The dispatcher takes femtotron's Column/RowParallelLinear at one rank
    (tensor_parallel/linear.py:42-64, 170-191: weight, bias, world_size,
    gather_output / scatter_input) and refuses them otherwise."""
    import torch
    from femtotron_amd.fused_checkpoint import _linear_weight

    class Col(torch.nn.Module):
        def __init__(self, ws=1, gather=False, bias=False):
            super().__init__()
            self.weight = torch.nn.Parameter(torch.zeros(4, 8))
            self.bias = torch.nn.Parameter(torch.zeros(4)) if bias else None
            self.world_size, self.rank, self.gather_output = ws, 0, gather

    class Row(torch.nn.Module):
        def __init__(self, ws=1, scatter=False):
            super().__init__()
            self.weight = torch.nn.Parameter(torch.zeros(8, 4))
            self.bias = None
            self.world_size, self.rank, self.scatter_input = ws, 0, scatter

    assert _linear_weight(Col()) is not None and _linear_weight(Row()) is not None
    assert _linear_weight(torch.nn.Linear(8, 4, bias=False)) is not None
    for bad in (Col(ws=2), Col(gather=True), Col(bias=True), Row(ws=2), Row(scatter=True),
                torch.nn.Linear(8, 4)):
        assert _linear_weight(bad) is None


def test_dispatch_table_routes_the_residual_form_by_its_own_entry():
    """The shipped table carries the four forms (nt, nn, tn and the down
    projection's residual form nt_res) and linear_residual consults nt_res."""
    import inspect
    import json

    from femtotron_amd import projections
    table = projections._library_shapes()
    assert set(table) == {"nt", "nn", "tn", "nt_res"}
    data = json.loads(projections.TABLE_FILE.read_text())
    measured = {(r["op"], r["m"], r["n"], r["k"]) for r in data["measurements"]}
    for op, shapes in table.items():
        for m, n, k in shapes:
            assert (op, m, n, k) in measured, (op, m, n, k)
    # every nt_res entry is a down projection (n = hidden, k = ffn) measured as such
    assert all(r["op"] != "nt_res" or (r["m"], r["n"], r["k"]) in {(m, n, k) for _, m, n, k in measured if _ == "nt"}
               for r in data["measurements"])
    assert '"nt_res"' in inspect.getsource(projections.linear_residual)


def test_default_gemm_policy_is_the_hand_written_kernel(monkeypatch):
    """Out of the box every projection GEMM the kernel supports runs on
    fh_gemm_bf16; the measured table is consulted only under policy 'auto'
    (operand checks stubbed: no device here, no kernel runs)."""
    import torch

    from femtotron_amd import ops, projections
    assert projections.gemm_policy() == "hand"
    monkeypatch.setattr(ops, "gemm_supported", lambda op, a, b: True)
    x = torch.empty(16384, 2048, dtype=torch.bfloat16, device="meta")
    w = torch.empty(11264, 2048, dtype=torch.bfloat16, device="meta")
    listed = ops.gemm_dims("nt", x, w) in projections._library_shapes()["nt"]
    assert listed, "the shipped table lists the TinyLlama gate/up forward GEMM"
    assert projections._choose_hand("nt", x, w)
    projections.set_gemm_policy("auto")
    try:
        assert not projections._choose_hand("nt", x, w)
    finally:
        projections.set_gemm_policy("hand")
