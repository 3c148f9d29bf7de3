"""Host side of the fused AdamW (femtotron_amd/optim.py): the tensor table's
layout matches FhAdamTensor/FhAdamHyper of include/femtohip.h, and the
optimizer refuses what the kernel cannot take (no GPU needed)."""
from __future__ import annotations

import ctypes

import pytest
import torch

from femtotron_amd._lib import FhAdamHyper
from femtotron_amd.optim import CHUNK, FusedAdamW, _Tensor, get_param_groups


def _c_layout() -> dict | None:
    """sizeof / offsetof of FhAdamTensor and FhAdamHyper as the C compiler lays
    them out from include/femtohip.h (None if no host compiler or ROCm headers)."""
    import shutil
    import subprocess
    import tempfile
    from pathlib import Path
    root = Path(__file__).resolve().parents[1]
    cc = shutil.which("gcc")
    if cc is None or not Path("/opt/rocm/include/hip/hip_runtime_api.h").exists():
        return None
    fields = ["param", "grad", "master", "exp_avg", "exp_avg_sq", "numel", "decay", "step_size",
              "bias_correction2_sqrt", "reserved"]
    src = ["#define __HIP_PLATFORM_AMD__ 1", "#include <stdio.h>", "#include <stddef.h>",
           '#include "femtohip.h"', "int main(void) {",
           '  printf("%zu %zu\\n", sizeof(FhAdamTensor), sizeof(FhAdamHyper));']
    src += [f'  printf("%zu\\n", offsetof(FhAdamTensor, {f}));' for f in fields]
    src += ["  return 0;", "}"]
    with tempfile.TemporaryDirectory() as d:
        c, exe = Path(d) / "layout.c", Path(d) / "layout"
        c.write_text("\n".join(src) + "\n")
        res = subprocess.run([cc, "-I", str(root / "include"), "-I", "/opt/rocm/include", str(c), "-o",
                              str(exe)], capture_output=True, text=True)
        if res.returncode != 0:
            return None
        out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()
    return {"tensor": int(out[0]), "hyper": int(out[1]), "offsets": dict(zip(fields, map(int, out[2:])))}


def test_table_layout_matches_header():
    fields = ["param", "grad", "master", "exp_avg", "exp_avg_sq", "numel", "decay", "step_size",
              "bias_correction2_sqrt", "reserved"]
    assert ctypes.sizeof(_Tensor) == 64
    assert [getattr(_Tensor, f).offset for f in fields] == [0, 8, 16, 24, 32, 40, 48, 52, 56, 60]
    assert ctypes.sizeof(FhAdamHyper) == 16
    assert CHUNK == 2048  # kAdamChunk of fh_adamw.hip: 256 threads x 8 elements
    c = _c_layout()
    if c is not None:  # the C compiler's layout of the same header
        assert c["tensor"] == ctypes.sizeof(_Tensor) and c["hyper"] == ctypes.sizeof(FhAdamHyper)
        assert c["offsets"] == {f: getattr(_Tensor, f).offset for f in fields}


def test_is_a_torch_optimizer():
    """Schedulers (the reference wraps its inner optimizer in LambdaLR) need a
    torch.optim.Optimizer with param_groups."""
    assert issubclass(FusedAdamW, torch.optim.Optimizer)


def test_rejects_host_parameters():
    with pytest.raises(ValueError, match="HIP device"):
        FusedAdamW([torch.zeros(8, requires_grad=True)])
    with pytest.raises(ValueError, match="HIP device"):
        FusedAdamW([{"params": [torch.zeros(8, dtype=torch.float64)], "weight_decay": 0.1}])


def test_param_groups_follow_the_reference_rule():
    """femtotron/training/optimizer.py:5-45: 1-D, "bias" and "embed" parameters
    take no weight decay."""
    from femtotron_amd.model import build_llama_model
    from tests.helpers import CFG1, llama_config
    model = build_llama_model(llama_config(CFG1))
    decay, no_decay = get_param_groups(model, 0.1)
    names = {id(p): n for n, p in model.named_parameters()}
    assert decay["weight_decay"] == 0.1 and no_decay["weight_decay"] == 0.0
    assert all(p.ndim == 2 and "embed" not in names[id(p)] for p in decay["params"])
    assert any("embed" in names[id(p)] for p in no_decay["params"])
    assert len(decay["params"]) + len(no_decay["params"]) == len(list(model.parameters()))
