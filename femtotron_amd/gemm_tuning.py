"""Tuned library GEMM selection for the layer's projections (hipBLASLt / rocBLAS).

The 7 projections of a decoder layer (femtotron/parallel/tensor_parallel/linear.py:66-80,
194-214 at TP=1) and the lm_head run as plain library GEMMs through ``torch.mm``
in three layouts: forward ``x @ W^T``, input gradient ``dY @ W`` and weight
gradient ``dY^T @ X``.  The library's default heuristic picks a kernel per shape;
for these shapes (M = tokens = 8k-32k, K = 2k-14k) an exhaustive search over
the hipBLASLt and rocBLAS solutions finds kernels up to 1.7x faster.

PyTorch's TunableOp performs that search and stores its choices as a CSV keyed
by (layout, m, n, k, leading dims), validated against the torch / HIP /
hipBLASLt / rocBLAS versions and the GPU architecture.  This module ships such
a file for gfx950 (``tuned/tunableop_gfx950.csv``, produced by ``tune()`` on an
MI355X for the workloads in ``WORKLOADS``) and turns it on:

    femtotron_amd.gemm_tuning.use_tuned_gemms()

Opt-in, because it switches a process-wide PyTorch setting: every ``torch.mm``
whose shape is in the file uses the recorded solution, every other GEMM keeps
the default heuristic; tuning itself stays off (no search at run time).  The
choice changes only the order of the fp32 accumulation inside a GEMM.
"""
from __future__ import annotations

import time
from pathlib import Path

import torch

TUNED_DIR = Path(__file__).resolve().parent / "tuned"
RESULTS_FILE = TUNED_DIR / "tunableop_gfx950.csv"

# (tokens, hidden, q width, kv width, ffn, vocab) of the benchmarked workloads:
# TinyLlama-1.1B at 8 x 2048 tokens, the Llama-3-8B slice at 1 x 8192 and the
# Llama-2-7B long-context slice at 1 x 32768.
WORKLOADS = {
    "tinyllama": (16384, 2048, 2048, 256, 5632, 32000),
    "llama3-8b-slice": (8192, 4096, 4096, 1024, 14336, 128256),
    "llama2-7b-long": (32768, 4096, 4096, 4096, 11008, 32000),
}


def use_tuned_gemms(path: str | Path | None = None) -> bool:
    """Serve ``torch.mm`` from the recorded solutions in ``path`` (default: the
    shipped gfx950 file).  Returns False, changing nothing, when the file is
    absent, no HIP device is present, or TunableOp rejects the file (its
    validators -- torch, HIP, hipBLASLt, rocBLAS versions and the GPU
    architecture -- do not match this process)."""
    path = Path(path) if path is not None else RESULTS_FILE
    if not path.is_file() or not torch.cuda.is_available():
        return False
    tunable = torch.cuda.tunable
    was_enabled = tunable.is_enabled()
    tunable.enable(True)
    tunable.tuning_enable(False)
    tunable.record_untuned_enable(False)
    tunable.set_filename(str(path))
    if not tunable.read_file(str(path)):
        tunable.enable(was_enabled)
        return False
    return True


def layer_gemm_shapes(workload: str) -> list[tuple[str, int, int]]:
    """(name, out features N, in features K) of every projection GEMM one step
    of `workload` issues: fused q/k/v, o, fused gate/up, down, lm_head (plus the
    separate projections of the selective / reference path)."""
    _, H, hq, hkv, F, V = WORKLOADS[workload]
    return [("qkv", hq + 2 * hkv, H), ("o", H, hq), ("gate_up", 2 * F, H), ("down", H, F),
            ("lm_head", V, H), ("q", hq, H), ("kv", hkv, H), ("gate", F, H)]


def tune(workloads=tuple(WORKLOADS), path: str | Path = RESULTS_FILE, *,
         max_ms_per_solution: int = 30, max_iters_per_solution: int = 10, log=print) -> Path:
    """Run TunableOp's search for every GEMM form of `workloads` (forward NT,
    input-gradient NN, weight-gradient TN; the lm_head, which is outside the
    layer, in its forward form only) and write the results CSV.  Needs a HIP
    device; each search takes seconds to a minute, one line is logged per GEMM."""
    tunable = torch.cuda.tunable
    tunable.enable(True)
    tunable.tuning_enable(True)
    tunable.record_untuned_enable(False)
    tunable.set_max_tuning_duration(max_ms_per_solution)
    tunable.set_max_tuning_iterations(max_iters_per_solution)
    tunable.set_filename(str(path))
    dev, bf = "cuda", torch.bfloat16
    g = torch.Generator(device=dev).manual_seed(0)
    for wl in workloads:
        T = WORKLOADS[wl][0]
        for name, N, K in layer_gemm_shapes(wl):
            x = torch.randn(T, K, device=dev, dtype=bf, generator=g)
            w = torch.randn(N, K, device=dev, dtype=bf, generator=g)
            dy = torch.randn(T, N, device=dev, dtype=bf, generator=g)
            forms = [("fwd x@W^T", lambda: torch.mm(x, w.t())),
                     ("dgrad dY@W", lambda: torch.mm(dy, w)),
                     ("wgrad dY^T@X", lambda: torch.mm(dy.t(), x))]
            for form, fn in forms[:1] if name == "lm_head" else forms:
                t0 = time.perf_counter()
                fn()
                torch.cuda.synchronize()
                log(f"[tune] {wl} {name} {form} T={T} N={N} K={K}: {time.perf_counter() - t0:.1f} s")
            del x, w, dy
    write_results(path)
    tunable.tuning_enable(False)
    return Path(path)


def write_results(path: str | Path) -> None:
    """Write TunableOp's validators and results in its own CSV format
    ("Validator,<key>,<value>" lines, then "<op>,<shape key>,<solution>,<ms>")."""
    lines = [f"Validator,{k},{v}" for k, v in torch.cuda.tunable.get_validators()]
    lines += [f"{op},{key},{sol},{ms}" for op, key, sol, ms in torch.cuda.tunable.get_results()]
    Path(path).write_text("\n".join(lines) + "\n")
