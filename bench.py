#!/usr/bin/env python
"""Benchmark: activation-checkpointed fwd+bwd tokens/s of the TinyLlama-1.1B-shaped
model on one MI355X, through the fused HIP checkpoint path.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload W] [--ac full|selective]

One step = forward (embed, 22 checkpointed decoder layers, final norm, lm_head,
shifted fp32 cross-entropy) + backward (per-layer recompute + layer backward)
over one synthetic micro-batch of 8 x 2048 token ids already resident in HBM.
The default workload is the metric's (TinyLlama, every layer checkpointed);
--workload llama3-8b-slice / llama2-7b-long run BASELINE configs 4 and 5 (an
8-layer Llama-3-8B slice at 1 x 8192 tokens, a 4-layer Llama-2-7B slice at
1 x 32768 tokens) and --ac selective the selective policy (MLP and norms
checkpointed) instead of whole layers.
Prints ONE JSON line.  Besides tokens/s it reports:
  * roofline: this build's dominant kernel, the hand-written kernel with the most
    time per step (a projection GEMM on fh_gemm_bf16 on the TinyLlama step), its
    algorithmic FLOPs (or bytes) per launch / its mean launch time (HIP events on
    the launch stream, the kernel alone at the step's shape) against the 2.5
    PFLOP/s dense bf16 MFMA peak (or the 8 TB/s HBM peak); roofline_hbm the same
    for the fused memory-bound kernel with the most time per step;
  * every fused memory-bound kernel against HBM peak at the step's shapes, and at
    BASELINE config 2's op-level shapes with the MALL flushed before each launch;
  * attention kernels and every projection GEMM (hand-written and library, the
    one the dispatch runs marked) against the MFMA peak; model and hardware FLOPs
    per token and the step's MFU / HFU;
  * peak activation bytes per token of the fused path and of the reference path
    (Hugging Face layers under torch.utils.checkpoint, debug=True as the
    reference's wrapper calls it, and debug=False) on the same GPU;
  * cpu_baseline: the reference-equivalent path (oracle/torch_llama.py under
    torch.utils.checkpoint with debug=True and debug=False, fp32) on the host
    cores, on a bounded sample of the same model, plus BASELINE configs 1 and 2.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

METRIC = "ckpt'd fwd+bwd tokens/s @1 GPU (TinyLlama-1.1B); fused-kernel HBM GB/s % of peak"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0

TINYLLAMA = dict(hidden=2048, heads=32, kv=4, ffn=5632, vocab=32000, layers=22, theta=10000.0,
                 batch=8, seq=2048)
WORKLOADS = {
    "tinyllama": (TINYLLAMA, "TinyLlama-1.1B", "BASELINE config 3"),
    "llama3-8b-slice": (dict(hidden=4096, heads=32, kv=8, ffn=14336, vocab=128256, layers=8,
                             theta=500000.0, batch=1, seq=8192), "Llama-3-8B 8-layer slice",
                        "BASELINE config 4"),
    "llama2-7b-long": (dict(hidden=4096, heads=32, kv=32, ffn=11008, vocab=32000, layers=4,
                            theta=10000.0, batch=1, seq=32768), "Llama-2-7B 4-layer slice, long context",
                       "BASELINE config 5"),
}
PRESETS = {"full": "llama_decoder_layer", "selective": "llama_mlp_and_norms"}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="tinyllama",
                    help="model shape (default: TinyLlama-1.1B, the metric's workload)")
    ap.add_argument("--ac", choices=sorted(PRESETS), default="full",
                    help="checkpointing policy: every decoder layer (full) or the MLP and norms "
                         "(selective)")
    ap.add_argument("--layers", type=int, default=None,
                    help="decoder layers (default: the workload's, 22 for TinyLlama-1.1B)")
    ap.add_argument("--kernel-iters", type=int, default=20)
    ap.add_argument("--reference-steps", type=int, default=2,
                    help="timed steps of the reference path on the GPU (0 to skip)")
    ap.add_argument("--cpu-sample-tokens", type=int, default=512,
                    help="tokens (one sequence) of the CPU baseline sample (0 to skip)")
    ap.add_argument("--stock-loss-head", action="store_true",
                    help="fused path with the reference's loss head (materialised fp32 logits) "
                         "instead of the fused lm_head + chunked cross-entropy")
    ap.add_argument("--no-tuned-gemms", action="store_true",
                    help="use the library's default GEMM heuristics instead of the shipped "
                         "TunableOp solutions (femtotron_amd/tuned/tunableop_gfx950.csv)")
    ap.add_argument("--tune-gemms", default=None, metavar="CSV",
                    help="run TunableOp's search for every projection GEMM of --workload, write "
                         "the results to CSV and exit")
    ap.add_argument("--gemm", choices=("hand", "auto", "library"), default="hand",
                    help="projection GEMMs: the hand-written fh_gemm_bf16 wherever it applies (the "
                         "default), the per-shape choice of the measured table "
                         "(femtotron_amd/tuned/gemm_dispatch_gfx950.json), or the library GEMM")
    ap.add_argument("--wgrad-stream", choices=("serial", "side"), default="serial",
                    help="weight-gradient GEMMs in series with the input-gradient chain (measured "
                         "faster with the hand-written GEMMs) or on a side stream next to it")
    ap.add_argument("--tune-gemm-dispatch", action="store_true",
                    help="time fh_gemm_bf16 against the library GEMM for every projection GEMM of "
                         "the three workloads, write femtotron_amd/tuned/gemm_dispatch_gfx950.json "
                         "and exit")
    ap.add_argument("--stock-boundary", action="store_true",
                    help="keep the reference's nn.Embedding and final LlamaRMSNorm (no fuse_boundary_ops)")
    ap.add_argument("--stock-attention", action="store_true",
                    help="under --ac selective keep HF's LlamaAttention outside the checkpoints "
                         "(no fuse_attention)")
    ap.add_argument("--no-auto-gemm-step", action="store_true",
                    help="under --gemm hand, skip the second timing of the step with the measured "
                         "table's routing (--gemm auto)")
    ap.add_argument("--no-chain", action="store_true",
                    help="skip the BASELINE config 2 op-level table of the memory-bound chain")
    ap.add_argument("--no-optimizer", action="store_true",
                    help="skip the fused-AdamW timing (reported beside the fwd+bwd metric)")
    ap.add_argument("--profile-kernel", default=None,
                    help="launch only this fused kernel (swiglu_fwd, swiglu_bwd, rmsnorm_fwd, "
                         "add_rmsnorm_fwd, rmsnorm_bwd, rope_fwd, residual_add, attn_fwd, attn_bwd; "
                         "embedding_fwd, embedding_bwd; gemm_<nt|nn|tn>_<qkv|o|gate_up|down> "
                         "(fh_gemm_bf16 at that projection GEMM; libgemm_...: the library GEMM); "
                         "adamw: one optimizer step over the workload's parameter shapes; "
                         "chain_cfg2: BASELINE config 2's memory-bound chain, each launch after a "
                         "MALL-evicting read) at "
                         "--workload's step shape, after a 1 GiB device copy that calibrates HBM byte "
                         "counters, for rocprofv3 --pmc runs; prints one JSON line and exits")
    return ap.parse_args()


def llama_config(c: dict, layers: int):
    from transformers import LlamaConfig
    cfg = LlamaConfig(hidden_size=c["hidden"], intermediate_size=c["ffn"],
                      num_attention_heads=c["heads"], num_key_value_heads=c["kv"],
                      num_hidden_layers=layers, vocab_size=c["vocab"], rms_norm_eps=1e-5,
                      hidden_act="silu", max_position_embeddings=max(2048, c["seq"]),
                      tie_word_embeddings=False, rope_theta=c["theta"], attention_dropout=0.0)
    cfg._attn_implementation = "sdpa"
    return cfg


def time_steps(torch, model, ids, steps: int, warmup: int, materialize_logits: bool = True) -> float:
    params = [p for p in model.parameters() if p.requires_grad]

    def step():
        for p in params:
            p.grad = None
        model(ids, labels=ids, materialize_logits=materialize_logits)["loss"].backward()

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def activation_bytes_per_token(torch, model, ids, materialize_logits: bool = True) -> float:
    """(max_memory_allocated during one fwd+bwd - memory_allocated before the
    forward) / tokens, with the gradients of a previous step already allocated
    (femtotron/test/integration/test_zero_ac.py:125-139 measures the same way)."""
    model(ids, labels=ids, materialize_logits=materialize_logits)["loss"].backward()  # grads exist
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    base = torch.cuda.memory_allocated()
    model(ids, labels=ids, materialize_logits=materialize_logits)["loss"].backward()
    torch.cuda.synchronize()
    return (torch.cuda.max_memory_allocated() - base) / ids.numel()


def measured_traffic(kernel: str):
    """HBM bytes per launch of `kernel` measured by rocprofv3 --pmc FETCH_SIZE and
    WRITE_SIZE runs (calibrated against a 1 GiB copy), as recorded in
    profiles/hbm_traffic.json; None if that kernel was not measured."""
    path = ROOT / "profiles" / "hbm_traffic.json"
    try:
        return json.loads(path.read_text())["kernels"][kernel]["traffic_bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def warm_up(torch, fn, ms: float = 40.0) -> None:
    """Launch fn() back to back for about `ms` milliseconds: under MFMA load
    the shader clock takes tens of milliseconds to settle (a cold first batch
    of attention-forward launches measured 225 us each, the same launches
    after 60 ms 176 us), so a kernel timed right after other work would be
    timed partly at a lower clock than it runs at inside the step."""
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    fn()
    end.record(stream)
    end.synchronize()
    n = max(1, int(ms / max(start.elapsed_time(end), 1e-3)))
    for _ in range(n):
        fn()
    torch.cuda.synchronize()


def event_ms(torch, fn, iters: int, warm: bool = False) -> float:
    """Mean launch time of fn() with HIP events on the current (launch) stream
    (after warm_up() when `warm`)."""
    fn()
    if warm:
        warm_up(torch, fn)
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for i in range(iters):
        fn(i)
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) / iters


def kernel_us(torch, fn, launches: int, before=None, sessions: int = 1) -> float:
    """Execution time of the kernels of this build that fn(i) launches (names
    in the fh:: namespace), per call, from the device timestamps torch.profiler
    collects (roctracer on ROCm: the kernel's own start and end, as
    rocprofv3 --kernel-trace reports them; launch gaps and host time are not
    included).  `launches` calls per profiling session, each preceded by
    before() if given; the median over `sessions` sessions of the per-call
    mean."""
    from torch.profiler import ProfilerActivity, profile
    fn(0)
    torch.cuda.synchronize()
    per = []
    for _ in range(sessions):
        with profile(activities=[ProfilerActivity.CUDA]) as prof:
            for i in range(launches):
                if before is not None:
                    before()
                fn(i)
            torch.cuda.synchronize()
        evs = [e for e in prof.events()
               if e.device_type == torch.autograd.DeviceType.CUDA and "fh::" in e.name]
        per.append(sum(e.device_time_total for e in evs) / launches)
    per.sort()
    return per[len(per) // 2]


def kernel_table(torch, c: dict, iters: int, ac: str, boundary: bool = True,
                 fused_attention: bool = False):
    """Fused kernels at the step's shapes.  Each launch reads a different buffer
    set (working set > 1 GiB) so the 256 MiB MALL cannot serve repeats: the bytes
    come from HBM as in the step.  launches_per_step counts the launches of one
    step of the model with c["layers"] layers under policy `ac`."""
    from femtotron_amd import ops
    T, H, F = c["batch"] * c["seq"], c["hidden"], c["ffn"]
    nh, nkv, hd = c["heads"], c["kv"], c["hidden"] // c["heads"]
    Hq, Hkv = nh * hd, nkv * hd
    dev = "cuda"
    bf = torch.bfloat16
    g = torch.Generator(device=dev).manual_seed(7)

    def rnd(*shape):
        return torch.randn(*shape, device=dev, dtype=bf, generator=g)

    def sets(n, make):
        return [make() for _ in range(n)]

    w = (1 + 0.02 * rnd(H)).contiguous()
    rows = []

    def add_row(name, kernel, launches_per_step, bytes_per_launch, ms, fn=None):
        # ms: HIP events around `iters` back-to-back launches (launch gaps
        # included); kernel_ms: the kernels' own execution time (fn re-run
        # under the profiler); achieved/frac from the latter
        kms = kernel_us(torch, fn, iters) / 1e3 if fn is not None else ms
        gbs = bytes_per_launch / (kms * 1e-3) / 1e9
        rows.append(dict(kernel=name, symbol=kernel, launches_per_step=launches_per_step,
                         bytes_per_launch=int(bytes_per_launch), ms_per_launch=round(kms, 5),
                         event_ms_per_launch=round(ms, 5),
                         achieved_gbs=round(gbs, 1), frac=round(gbs / HBM_PEAK_GBS, 4)))

    L = c["layers"]
    sel = ac == "selective"
    # attention's kernels run in the step: inside the fused layer (full AC,
    # forward twice: forward and recompute) or in fused_attention's modules
    # outside the checkpoints (selective AC, forward once)
    attn = not sel or fused_attention
    n_fwd = L if sel else 2 * L
    # rmsnorm_fwd: x -> y   (4TH bytes)
    xs = sets(8, lambda: rnd(T, H))
    ys = sets(8, lambda: torch.empty(T, H, device=dev, dtype=bf))
    rs = torch.empty(T, device=dev, dtype=torch.float32)
    f = lambda i=0: ops.rmsnorm_fwd(xs[i % 8], w, 1e-5, out=ys[i % 8], rstd=rs)
    ms = event_ms(torch, f, iters)
    # + the final norm: checkpointed under the selective policy, FusedRMSNorm otherwise
    add_row("rmsnorm_fwd", "k_rmsnorm_fwd", 2 * L + (1 if sel or boundary else 0), 4 * T * H, ms, f)
    # add_rmsnorm_fwd: x, a -> h, y   (8TH)
    as_ = sets(8, lambda: rnd(T, H))
    f = lambda i=0: ops.add_rmsnorm_fwd(xs[i % 8], as_[i % 8], w, 1e-5, rstd=rs)
    ms = event_ms(torch, f, iters)
    if not sel:
        add_row("add_rmsnorm_fwd", "k_rmsnorm_fwd (ADD)", 2 * L, 8 * T * H, ms, f)
    if sel:
        # rmsnorm_bwd without residual, statistic recomputed: dy, x -> dx   (6TH)
        f = lambda i=0: ops.rmsnorm_bwd(ys[i % 8], xs[i % 8], w, 1e-5)
        ms = event_ms(torch, f, iters)
        add_row("rmsnorm_bwd", "k_rmsnorm_bwd + k_reduce_parts", 2 * L + 1, 6 * T * H, ms, f)
    else:
        # rmsnorm_bwd with residual: dy, x, dres -> dx   (8TH)
        f = lambda i=0: ops.rmsnorm_bwd(ys[i % 8], xs[i % 8], w, 1e-5, rstd=rs, dres=as_[i % 8])
        ms = event_ms(torch, f, iters)
        add_row("rmsnorm_bwd", "k_rmsnorm_bwd + k_reduce_parts", 2 * L, 8 * T * H, ms, f)
        if boundary:
            # the final norm's backward: no residual, statistic recomputed: dy, x -> dx   (6TH)
            f = lambda i=0: ops.rmsnorm_bwd(ys[i % 8], xs[i % 8], w, 1e-5)
            ms = event_ms(torch, f, iters)
            add_row("final_rmsnorm_bwd", "k_rmsnorm_bwd + k_reduce_parts", 1, 6 * T * H, ms, f)
    del as_
    if not sel:
        # residual add: h + m -> out   (6TH)
        f = lambda i=0: ops.add(xs[i % 8], ys[i % 8], out=ys[(i + 1) % 8])
        ms = event_ms(torch, f, iters)
        add_row("residual_add", "k_add", L, 6 * T * H, ms, f)
    del xs, ys
    # rope on the k heads of the qkv buffer   (4T Hkv)
    qkvs = sets(6, lambda: rnd(T, Hq + 2 * Hkv))
    cos = torch.cos(torch.arange(c["seq"] * hd, device=dev, dtype=torch.float32)).to(bf).view(1, c["seq"], hd)
    sin = torch.sin(torch.arange(c["seq"] * hd, device=dev, dtype=torch.float32)).to(bf).view(1, c["seq"], hd)
    if attn:
        # k heads only: q is rotated as the attention forward loads it, and the
        # RoPE backward runs inside the attention backward's dQ / dK stores
        f = lambda i=0: ops.rope_fwd_(qkvs[i % 6][:, Hq:], nkv, hd, c["seq"], cos, sin)
        ms = event_ms(torch, f, iters)
        add_row("rope_fwd", "k_rope<fwd> (k heads)", n_fwd, 4 * T * Hkv, ms, f)
    # SwiGLU: g,u -> p (6TF), in the forward only (the recompute stops at the
    # gate/up projection);  dp,g,u -> dg,du and p over dp (12TF)
    gus = sets(3, lambda: rnd(T, 2 * F))
    ps = sets(3, lambda: torch.empty(T, F, device=dev, dtype=bf))
    f = lambda i=0: ops.swiglu_fwd(gus[i % 3][:, :F], gus[i % 3][:, F:], out=ps[i % 3])
    ms = event_ms(torch, f, iters)
    add_row("swiglu_fwd", "k_swiglu_fwd", L, 6 * T * F, ms, f)
    dgus = sets(3, lambda: torch.empty(T, 2 * F, device=dev, dtype=bf))
    f = lambda i=0: ops.swiglu_bwd(ps[i % 3], gus[i % 3][:, :F], gus[i % 3][:, F:],
                                   dgus[i % 3][:, :F], dgus[i % 3][:, F:], p_out=ps[i % 3])
    ms = event_ms(torch, f, iters)
    add_row("swiglu_bwd", "k_swiglu_bwd (+ p over dp)", L, 12 * T * F, ms, f)
    del gus, ps, dgus
    if boundary:
        # embedding: gather (T rows read and written + int64 ids); backward:
        # dy read, every vocabulary row written, ids read (the radix sort's
        # 4-byte keys/values are not counted)
        V = c["vocab"]
        emb = rnd(V, H)
        ids = torch.randint(0, V, (T,), device=dev, generator=g)
        f = lambda i=0: ops.embedding_fwd(ids, emb)
        ms = event_ms(torch, f, iters)
        add_row("embedding_fwd", "k_embed_fwd", 1, 4 * T * H + 8 * T, ms, f)
        dys = sets(3, lambda: rnd(T, H))
        f = lambda i=0: ops.embedding_bwd(dys[i % 3], ids, V)
        ms = event_ms(torch, f, iters)
        add_row("embedding_bwd", "k_embed_keys + 3 x k_radix_* + k_embed_bounds + k_embed_rows", 1,
                2 * T * H + 2 * V * H + 8 * T, ms, f)
        del emb, dys
    if not attn:  # HF's attention outside the checkpointed modules (selective, --stock-attention)
        return rows, []

    # attention (MFMA-bound): causal flop count 4*B*nh*S^2*hd/2 forward
    B, S = c["batch"], c["seq"]
    qkv = qkvs[0]
    q, k, v = qkv[:, :Hq], qkv[:, Hq:Hq + Hkv], qkv[:, Hq + Hkv:]
    fwd_flop = 4 * B * nh * S * S * hd / 2
    o, lse = ops.attn_fwd(q, k, v, B, S, nh, nkv, hd, hd ** -0.5)
    # the recompute's form: q rotated on load and written out rotated for the backward
    q_rot = torch.empty_like(q)
    ms_f = event_ms(torch, lambda i=0: ops.attn_fwd(q, k, v, B, S, nh, nkv, hd, hd ** -0.5, rope=(cos, sin),
                                                      q_out=q_rot), iters, warm=True)
    do = rnd(T, Hq)
    dqkv = torch.empty_like(qkv)
    ms_b = event_ms(torch, lambda i=0: ops.attn_bwd(q, k, v, o, do, lse, dqkv[:, :Hq], dqkv[:, Hq:Hq + Hkv],
                                                      dqkv[:, Hq + Hkv:], B, S, nh, nkv, hd, hd ** -0.5,
                                                      rope=(cos, sin)),
                    iters, warm=True)
    # backward: dK/dV kernel 4 products + dQ kernel 3 products (the dQ kernel
    # recomputes S and dP); algorithmic = the 5 products of attention backward
    bwd_flop = 2.5 * fwd_flop
    # The reference's own kernel at the same shapes: torch's SDPA, causal, GQA
    # (HF integrations/sdpa_attention.py:154-163), on [B, heads, S, hd]
    # tensors; forward, and forward + backward (autograd.grad, so no
    # accumulation into .grad), the backward taken as their difference.
    import torch.nn.functional as Fn
    gqa = nkv != nh
    qh = q.reshape(B, S, nh, hd).transpose(1, 2).contiguous()
    kh = k.reshape(B, S, nkv, hd).transpose(1, 2).contiguous()
    vh = v.reshape(B, S, nkv, hd).transpose(1, 2).contiguous()
    doh = do.reshape(B, S, nh, hd).transpose(1, 2).contiguous()

    def sdpa(a, b_, c_):
        return Fn.scaled_dot_product_attention(a, b_, c_, is_causal=True, scale=hd ** -0.5, enable_gqa=gqa)

    lib_f = event_ms(torch, lambda i=0: sdpa(qh, kh, vh), iters, warm=True)
    qg, kg, vg = (t.detach().requires_grad_(True) for t in (qh, kh, vh))
    lib_fb = event_ms(torch, lambda i=0: torch.autograd.grad(sdpa(qg, kg, vg), (qg, kg, vg), doh),
                      max(3, iters // 4), warm=True)
    lib_b = max(lib_fb - lib_f, 1e-6)
    del qh, kh, vh, doh, qg, kg, vg
    lib_note = "torch.nn.functional.scaled_dot_product_attention(is_causal=True, enable_gqa) at the same shape"
    mfma = [dict(kernel="attn_fwd", symbol=f"k_attn_fwd<{hd}>, q rotated on load and written out "
                                           "(fh_attn_fwd_rope)", launches_per_step=n_fwd,
                 flop_per_launch=fwd_flop, ms_per_launch=round(ms_f, 4),
                 achieved_tflops=round(fwd_flop / ms_f / 1e9, 1),
                 frac=round(fwd_flop / ms_f / 1e9 / MFMA_BF16_PEAK_TFLOPS, 4),
                 library_ms=round(lib_f, 4), library=lib_note + " (forward; the library's forward does "
                                                                "no RoPE)"),
            dict(kernel="attn_bwd", symbol=f"k_attn_bwd_dq<{hd}> + k_attn_bwd_dkdv"
                                           f"{'_fused' if hd <= 64 else ''}<{hd}>, RoPE backward in the "
                                           "dQ / dK stores (fh_attn_bwd_rope)",
                 launches_per_step=L, flop_per_launch=bwd_flop, ms_per_launch=round(ms_b, 4),
                 achieved_tflops=round(bwd_flop / ms_b / 1e9, 1),
                 frac=round(bwd_flop / ms_b / 1e9 / MFMA_BF16_PEAK_TFLOPS, 4),
                 library_ms=round(lib_b, 4), library=lib_note + " (forward + backward less forward; "
                                                                "no RoPE)")]
    mfma += projection_gemm_rows(torch, c, iters, sel, fused_attention, rnd)
    return rows, mfma


# the decoder layer's memory-bound chain, op-level.
CHAIN_CFG2 = dict(tokens=4096, hidden=4096, ffn=14336, rope_heads=32, head_dim=128, theta=500000.0)
MALL_FLUSH_BYTES = 512 << 20


def flushed_ms(torch, fn, reps: int, flush) -> float:
    """Median launch time of fn(i) over `reps` launches, each preceded by a
    read of a 512 MiB buffer (more than the 256 MiB MALL, so every launch's
    operands come from HBM); HIP events around each launch alone."""
    fn(0)
    stream = torch.cuda.current_stream()
    ev = []
    for i in range(reps):
        flush()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        fn(i)
        b.record(stream)
        ev.append((a, b))
    torch.cuda.synchronize()
    ms = sorted(a.elapsed_time(b) for a, b in ev)
    return ms[len(ms) // 2]


def chain_table(torch, shape: dict, reps: int) -> list:
    """The fused memory-bound kernels at BASELINE config 2's shapes (x [1, T, H]
    bf16, RMSNorm weight 1 + N(0, 0.02), RoPE on rope_heads x head_dim of q,
    SwiGLU gate/up [1, T, F], residual add; forward, recompute and backward
    kernels), inputs from CPU generators with seeds 1-5 as the op-level config
    prescribes, the MALL flushed before every launch."""
    from femtotron_amd import ops
    T, H, Fd = shape["tokens"], shape["hidden"], shape["ffn"]
    nr, hd = shape["rope_heads"], shape["head_dim"]
    dev, bf = "cuda", torch.bfloat16

    def cpu_randn(seed, *size):
        return torch.randn(*size, generator=torch.Generator().manual_seed(seed)).to(device=dev, dtype=bf)

    x = cpu_randn(1, T, H)
    w = (1 + 0.02 * torch.randn(H, generator=torch.Generator().manual_seed(2))).to(device=dev, dtype=bf)
    g = cpu_randn(3, T, Fd)
    u = cpu_randn(4, T, Fd)
    dy = cpu_randn(5, T, H)
    dp = cpu_randn(5, T, Fd)
    flush_buf = torch.ones(MALL_FLUSH_BYTES // 4, device=dev, dtype=torch.float32)

    def flush():
        flush_buf.sum()

    y = torch.empty_like(x)
    hh = torch.empty_like(x)
    rs = torch.empty(T, device=dev, dtype=torch.float32)
    q = x[:, :nr * hd].clone()
    inv = 1.0 / (shape["theta"] ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd))
    ang = torch.arange(T, dtype=torch.float32)[:, None] * inv[None, :]
    ang = torch.cat((ang, ang), dim=-1)[None]
    cos, sin = ang.cos().to(device=dev, dtype=bf), ang.sin().to(device=dev, dtype=bf)
    p = torch.empty(T, Fd, device=dev, dtype=bf)
    dg, du = torch.empty_like(p), torch.empty_like(p)
    rows = []

    def row(name, symbol, nbytes, fn):
        # kernel-only time (profiler, one launch per session after the flush,
        # median) and the HIP-event time around the launch for comparison
        ms = kernel_us(torch, fn, 1, before=flush, sessions=reps) / 1e3
        ev = flushed_ms(torch, fn, reps, flush)
        gbs = nbytes / (ms * 1e-3) / 1e9
        rows.append(dict(kernel=name, symbol=symbol, bytes_per_launch=int(nbytes), ms_per_launch=round(ms, 5),
                         event_ms_per_launch=round(ev, 5),
                         achieved_gbs=round(gbs, 1), frac=round(gbs / HBM_PEAK_GBS, 4)))

    row("rmsnorm_fwd", "k_rmsnorm_fwd", 4 * T * H, lambda i: ops.rmsnorm_fwd(x, w, 1e-5, out=y, rstd=rs))
    row("add_rmsnorm_fwd", "k_rmsnorm_fwd (ADD)", 8 * T * H,
        lambda i: ops.add_rmsnorm_fwd(x, dy, w, 1e-5, rstd=rs))
    row("rmsnorm_bwd", "k_rmsnorm_bwd (+ residual gradient)", 8 * T * H,
        lambda i: ops.rmsnorm_bwd(dy, x, w, 1e-5, rstd=rs, dres=y))
    row("rmsnorm_bwd_plain", "k_rmsnorm_bwd", 6 * T * H, lambda i: ops.rmsnorm_bwd(dy, x, w, 1e-5))
    row("rope_fwd", "k_rope<fwd>", 4 * T * nr * hd, lambda i: ops.rope_fwd_(q, nr, hd, T, cos, sin))
    row("rope_bwd", "k_rope<bwd>", 4 * T * nr * hd, lambda i: ops.rope_bwd_(q, nr, hd, T, cos, sin))
    row("swiglu_fwd", "k_swiglu_fwd", 6 * T * Fd, lambda i: ops.swiglu_fwd(g, u, out=p))
    row("swiglu_bwd", "k_swiglu_bwd (+ p over dp)", 12 * T * Fd,
        lambda i: ops.swiglu_bwd(dp, g, u, dg, du, p_out=dp))
    row("residual_add", "k_add", 6 * T * H, lambda i: ops.add(x, dy, out=hh))
    # Practical ceiling at these sizes: torch's device-to-device copy of x
    # (T H bf16 read and written: the bytes of rmsnorm_fwd), cold as above.
    from torch.profiler import ProfilerActivity, profile
    cp = []
    for _ in range(reps):
        flush()
        with profile(activities=[ProfilerActivity.CUDA]) as prof:
            hh.copy_(x)
            torch.cuda.synchronize()
        cp.append(sum(e.device_time_total for e in prof.events()
                      if e.device_type == torch.autograd.DeviceType.CUDA and "Memcpy" in e.name) / 1e3)
    cp.sort()
    ms = cp[len(cp) // 2]
    if ms > 0:
        gbs = 4 * T * H / (ms * 1e-3) / 1e9
        rows.append(dict(kernel="device_copy (calibration)", symbol="torch copy_ (hipMemcpy device to device)",
                         bytes_per_launch=4 * T * H, ms_per_launch=round(ms, 5), achieved_gbs=round(gbs, 1),
                         frac=round(gbs / HBM_PEAK_GBS, 4)))
    del flush_buf
    return rows


def step_flops_per_token(c: dict) -> dict:
    """Algorithmic FLOPs per token of one step: the layer forward (projection
    GEMMs + causal attention 2 Hq S), counted 3x without recompute (model FLOPs)
    and 4x with the full-layer recompute (hardware FLOPs, the recompute path
    re-runs the layer up to SwiGLU, so the down projection is not counted
    twice), plus the lm_head 3x."""
    H, Fd, S = c["hidden"], c["ffn"], c["seq"]
    hd = H // c["heads"]
    Hq, Hkv = c["heads"] * hd, c["kv"] * hd
    gemm = 2 * (H * (Hq + 2 * Hkv) + Hq * H + 3 * H * Fd)
    attn = 2 * Hq * S
    fwd = gemm + attn
    head = 2 * H * c["vocab"]
    L = c["layers"]
    model = L * 3 * fwd + 3 * head
    hardware = L * (4 * fwd - 2 * H * Fd) + 3 * head
    return {"model": model, "hardware": hardware}


def projection_gemm_rows(torch, c: dict, iters: int, sel: bool, fused_attention: bool, rnd) -> list:
    """Every projection GEMM of the step at its shape: the hand-written
    fh_gemm_bf16 and the library GEMM timed side by side (HIP events), the one
    the dispatch policy runs marked `path`, its MFMA fraction in `frac`."""
    from femtotron_amd import ops, projections
    T, H, F, L = c["batch"] * c["seq"], c["hidden"], c["ffn"], c["layers"]
    hd = H // c["heads"]
    Hq, Hkv = c["heads"] * hd, c["kv"] * hd
    # launches per step: full AC runs the q/k/v, o and gate/up forward twice
    # (forward and recompute) and down once; selective AC recomputes the MLP's
    # gate/up only (attention runs once, outside the checkpoints)
    projs = [("qkv", Hq + 2 * Hkv, H, 1 if sel else 2), ("o", H, Hq, 1 if sel else 2),
             ("gate_up", 2 * F, H, 2), ("down", H, F, 1)]
    out = []
    for name, n_out, k_in, fwd_per_layer in projs:
        if sel and not fused_attention and name in ("qkv", "o"):
            continue
        x, w, dy = rnd(T, k_in), rnd(n_out, k_in), rnd(T, n_out)
        flop = 2 * T * n_out * k_in
        for op, a, b, lib, per_layer in (("nt", x, w, lambda: torch.mm(x, w.t()), fwd_per_layer),
                                         ("nn", dy, w, lambda: torch.mm(dy, w), 1),
                                         ("tn", dy, x, lambda: torch.mm(dy.t(), x), 1)):
            # the down projection's forward is linear_residual: the hand-written
            # GEMM's residual epilogue against the library GEMM + fh_add
            res = op == "nt" and name == "down"
            if res:
                r_, o_ = rnd(T, n_out), torch.empty(T, n_out, device=x.device, dtype=x.dtype)
                ms_hand = event_ms(torch, lambda i=0: ops.gemm(op, a, b, residual=r_, out=o_), iters, warm=True)
                ms_lib = event_ms(torch, lambda i=0: ops.add(r_, lib(), out=o_), iters, warm=True)
            else:
                ms_hand = event_ms(torch, lambda i=0: ops.gemm(op, a, b), iters, warm=True)
                ms_lib = event_ms(torch, lambda i=0: lib(), iters, warm=True)
            hand = projections.gemm_policy() != "library" and (
                projections.gemm_policy() == "hand"
                or ops.gemm_dims(op, a, b) not in projections._library_shapes()["nt_res" if res else op])
            ms = ms_hand if hand else ms_lib
            out.append(dict(kernel=f"gemm_{op}_{name}", m_n_k=list(ops.gemm_dims(op, a, b)),
                            path=("fh_gemm_bf16 (k_gemm)" if hand else "library (torch.mm)")
                            + (" with the residual add (epilogue / fh_add)" if res else ""),
                            launches_per_step=per_layer * L, flop_per_launch=flop,
                            ms_per_launch=round(ms, 4), hand_ms=round(ms_hand, 4),
                            library_ms=round(ms_lib, 4),
                            achieved_tflops=round(flop / ms / 1e9, 1),
                            frac=round(flop / ms / 1e9 / MFMA_BF16_PEAK_TFLOPS, 4)))
        del x, w, dy
    return out


def profile_kernel(torch, name: str, c: dict, launches: int = 10) -> dict:
    """A 1 GiB device-to-device copy (known traffic: 1 GiB read + 1 GiB written),
    then `launches` launches of one fused kernel at the step's shape of workload
    `c`, each on a fresh buffer set (attention: on one buffer set; chain_cfg2:
    BASELINE config 2's chain, each launch after a MALL-evicting read).  Under
    rocprofv3 --pmc FETCH_SIZE (or WRITE_SIZE) the copy's reading calibrates the
    counter's units."""
    from femtotron_amd import ops
    T, H, F = c["batch"] * c["seq"], c["hidden"], c["ffn"]
    nh, nkv, hd = c["heads"], c["kv"], c["hidden"] // c["heads"]
    Hq, Hkv = nh * hd, nkv * hd
    dev, bf = "cuda", torch.bfloat16
    g = torch.Generator(device=dev).manual_seed(3)

    def rnd(*shape):
        return torch.randn(*shape, device=dev, dtype=bf, generator=g)

    src = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    n = launches
    if name in ("swiglu_fwd", "swiglu_bwd"):
        gus = [rnd(T, 2 * F) for _ in range(n)]
        if name == "swiglu_fwd":
            fn = lambda i: ops.swiglu_fwd(gus[i][:, :F], gus[i][:, F:])
            nbytes = 6 * T * F
        else:
            dps = [rnd(T, F) for _ in range(n)]
            out = torch.empty(T, 2 * F, device=dev, dtype=bf)
            fn = lambda i: ops.swiglu_bwd(dps[i], gus[i][:, :F], gus[i][:, F:], out[:, :F], out[:, F:],
                                          p_out=dps[i])
            nbytes = 12 * T * F
    elif name in ("rmsnorm_fwd", "add_rmsnorm_fwd", "rmsnorm_bwd", "residual_add"):
        xs = [rnd(T, H) for _ in range(n)]
        as_ = [rnd(T, H) for _ in range(n)]
        w = (1 + 0.02 * rnd(H)).contiguous()
        fn = {"rmsnorm_fwd": lambda i: ops.rmsnorm_fwd(xs[i], w, 1e-5),
              "add_rmsnorm_fwd": lambda i: ops.add_rmsnorm_fwd(xs[i], as_[i], w, 1e-5),
              "rmsnorm_bwd": lambda i: ops.rmsnorm_bwd(as_[i], xs[i], w, 1e-5, dres=as_[(i + 1) % n]),
              "residual_add": lambda i: ops.add(xs[i], as_[i])}[name]
        nbytes = {"rmsnorm_fwd": 4, "add_rmsnorm_fwd": 8, "rmsnorm_bwd": 8, "residual_add": 6}[name] * T * H
    elif name == "rope_fwd":  # the k heads (q is rotated by the attention forward)
        qkvs = [rnd(T, Hq + 2 * Hkv) for _ in range(n)]
        cos = rnd(1, c["seq"], hd)
        sin = rnd(1, c["seq"], hd)
        fn = lambda i: ops.rope_fwd_(qkvs[i][:, Hq:], nkv, hd, c["seq"], cos, sin)
        nbytes = 4 * T * Hkv
    elif name in ("attn_fwd", "attn_bwd"):
        qkv = rnd(T, Hq + 2 * Hkv)
        q, k, v = qkv[:, :Hq], qkv[:, Hq:Hq + Hkv], qkv[:, Hq + Hkv:]
        o, lse = ops.attn_fwd(q, k, v, c["batch"], c["seq"], nh, nkv, hd, hd ** -0.5)
        do = rnd(T, Hq)
        dqkv = torch.empty_like(qkv)
        if name == "attn_fwd":
            cos = rnd(1, c["seq"], hd)
            sin = rnd(1, c["seq"], hd)
            q_rot = torch.empty_like(q)
            fn = lambda i: ops.attn_fwd(q, k, v, c["batch"], c["seq"], nh, nkv, hd, hd ** -0.5, rope=(cos, sin),
                                        q_out=q_rot)
        else:
            cos = rnd(1, c["seq"], hd)
            sin = rnd(1, c["seq"], hd)
            fn = lambda i: ops.attn_bwd(q, k, v, o, do, lse, dqkv[:, :Hq], dqkv[:, Hq:Hq + Hkv],
                                        dqkv[:, Hq + Hkv:], c["batch"], c["seq"], nh, nkv, hd, hd ** -0.5,
                                        rope=(cos, sin))
        nbytes = None
    elif name in ("embedding_fwd", "embedding_bwd"):
        V = c["vocab"]
        emb = rnd(V, H)
        ids = torch.randint(0, V, (T,), device=dev, generator=g)
        if name == "embedding_fwd":
            fn = lambda i: ops.embedding_fwd(ids, emb)
            nbytes = 4 * T * H + 8 * T
        else:
            dys = [rnd(T, H) for _ in range(n)]
            fn = lambda i: ops.embedding_bwd(dys[i], ids, V)
            nbytes = 2 * T * H + 2 * V * H + 8 * T
    elif name.startswith("gemm_") or name.startswith("libgemm_"):
        # gemm_<op>_<proj>: fh_gemm_bf16; libgemm_<op>_<proj>: the library GEMM
        # (torch.mm, with the shipped TunableOp solutions) at the same shape
        lib_, op, proj = name.split("_", 2)
        n_out, k_in = {"qkv": (Hq + 2 * Hkv, H), "o": (H, Hq), "gate_up": (2 * F, H),
                       "down": (H, F)}[proj]
        xs = [rnd(T, k_in) for _ in range(2)]
        ws = [rnd(n_out, k_in) for _ in range(2)]
        dys = [rnd(T, n_out) for _ in range(2)]
        operands = {"nt": (xs, ws), "nn": (dys, ws), "tn": (dys, xs)}[op]
        if lib_ == "libgemm":
            mm = {"nt": lambda a, b: torch.mm(a, b.t()), "nn": torch.mm, "tn": lambda a, b: torch.mm(a.t(), b)}[op]
            fn = lambda i: mm(operands[0][i % 2], operands[1][i % 2])
        else:
            fn = lambda i: ops.gemm(op, operands[0][i % 2], operands[1][i % 2])
        nbytes = None  # MFMA-bound: 2*T*n_out*k_in FLOP per launch
    elif name == "chain_cfg2":
        # BASELINE config 2's memory-bound chain, each kernel `launches` times,
        # every launch after a 512 MiB read that evicts the MALL (the launches
        # of chain_table, without its profiler or events)
        sh = CHAIN_CFG2
        Tc, Hc, Fc, nr, hdc = sh["tokens"], sh["hidden"], sh["ffn"], sh["rope_heads"], sh["head_dim"]
        x, dy, hh = rnd(Tc, Hc), rnd(Tc, Hc), torch.empty(Tc, Hc, device=dev, dtype=bf)
        w = (1 + 0.02 * rnd(Hc)).contiguous()
        gg, uu, dp = rnd(Tc, Fc), rnd(Tc, Fc), rnd(Tc, Fc)
        dg, du, pp = (torch.empty(Tc, Fc, device=dev, dtype=bf) for _ in range(3))
        q = rnd(Tc, nr * hdc)
        cos, sin = rnd(1, Tc, hdc), rnd(1, Tc, hdc)
        rs = torch.empty(Tc, device=dev, dtype=torch.float32)
        ops.rmsnorm_fwd(x, w, 1e-5, out=hh, rstd=rs)
        flush_buf = torch.ones(MALL_FLUSH_BYTES // 4, device=dev, dtype=torch.float32)
        chain = [lambda: ops.rmsnorm_fwd(x, w, 1e-5, out=hh, rstd=rs),
                 lambda: ops.add_rmsnorm_fwd(x, dy, w, 1e-5, rstd=rs),
                 lambda: ops.rmsnorm_bwd(dy, x, w, 1e-5, rstd=rs, dres=hh),
                 lambda: ops.rmsnorm_bwd(dy, x, w, 1e-5),
                 lambda: ops.rope_fwd_(q, nr, hdc, Tc, cos, sin),
                 lambda: ops.rope_bwd_(q, nr, hdc, Tc, cos, sin),
                 lambda: ops.swiglu_fwd(gg, uu, out=pp),
                 lambda: ops.swiglu_bwd(dp, gg, uu, dg, du, p_out=dp),
                 lambda: ops.add(x, dy, out=hh)]

        def fn(i):
            for f in chain:
                flush_buf.sum()
                f()
        nbytes = None
    elif name == "adamw":
        from femtotron_amd.optim import FusedAdamW
        V, L = c["vocab"], c["layers"]
        shapes = [(V, H)] + [(Hq, H), (Hkv, H), (Hkv, H), (H, Hq), (F, H), (F, H), (H, F), (H,), (H,)] * L
        shapes += [(H,), (V, H)]
        params = [rnd(*s) for s in shapes]
        for p in params:
            p.grad = rnd(*p.shape)
        opt = FusedAdamW([{"params": [p for p in params if p.dim() > 1], "weight_decay": 0.01},
                          {"params": [p for p in params if p.dim() == 1], "weight_decay": 0.0}],
                         lr=3e-4, max_grad_norm=1.0)
        fn = lambda i: opt.step()
        nbytes = 30 * sum(p.numel() for p in params)  # per step: k_grad_sq 2 B, k_adamw 28 B per param
    else:
        raise SystemExit(f"unknown kernel {name!r}")
    torch.cuda.synchronize()
    for i in range(n):
        fn(i)
    torch.cuda.synchronize()
    return {"profile_kernel": name, "launches": n, "algorithmic_bytes_per_launch": nbytes,
            "calibration_copy_bytes": 1 << 30, "shape": {"tokens": T, "hidden": H, "ffn": F}}


def optimizer_timing(torch, model, iters: int) -> dict:
    """The mixed-precision AdamW step over the model's parameters with random
    bf16 gradients: the fused path (FusedAdamW, one fh_adamw_step call) against
    the reference's sequence on the same GPU (master.grad = grad.float();
    ClipGradNorm; torch.optim.AdamW(foreach) on the fp32 masters;
    param.copy_(master)).  Algorithmic bytes per bf16 parameter: 2 (gradient,
    norm pass) + 2 + 3 x 4 read (gradient, master, moments) + 3 x 4 + 2 written
    = 30."""
    from femtotron_amd.optim import FusedAdamW, get_param_groups
    params = list(model.parameters())
    gen = torch.Generator(device="cuda").manual_seed(11)
    for p in params:
        p.grad = torch.randn(p.shape, device=p.device, dtype=p.dtype, generator=gen)
    n = sum(p.numel() for p in params)
    kw = dict(lr=3e-4, betas=(0.9, 0.95), eps=1e-8)
    opt = FusedAdamW(get_param_groups(model, 0.01), max_grad_norm=1.0, **kw)
    ms = event_ms(torch, lambda i=0: opt.step(), iters)
    del opt
    torch.cuda.empty_cache()
    masters = {id(p): p.detach().float().clone().requires_grad_(True) for p in params}
    groups = [{"params": [masters[id(p)] for p in g["params"]], "weight_decay": g["weight_decay"]}
              for g in get_param_groups(model, 0.01)]
    ref = torch.optim.AdamW(groups, foreach=True, **kw)

    def ref_step(i=0):
        for p in params:
            masters[id(p)].grad = p.grad.float()
        grads = [m.grad for m in masters.values()]
        total = torch.zeros((), device="cuda")
        for g in grads:
            total += g.float().pow(2).sum()
        coef = (1.0 / (total.sqrt() + 1e-6)).clamp(max=1.0)
        for g in grads:
            g.mul_(coef)
        ref.step()
        with torch.no_grad():
            for p in params:
                p.copy_(masters[id(p)])

    ms_ref = event_ms(torch, ref_step, max(3, iters // 4))
    del ref, masters, groups
    for p in params:
        p.grad = None
    torch.cuda.empty_cache()
    gbs = 30 * n / (ms * 1e-3) / 1e9
    return {"kernels": "k_grad_sq + k_clip_coef + k_adamw (one fh_adamw_step call)", "params": n,
            "bytes_per_step": 30 * n, "ms_per_step": round(ms, 4), "achieved_gbs": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4), "reference_ms_per_step": round(ms_ref, 3),
            "speedup_vs_reference": round(ms_ref / ms, 2),
            "reference": "master.grad = grad.float(); ClipGradNorm(1.0); torch.optim.AdamW(foreach) "
                         "on fp32 masters; param.copy_(master)"}


def host_info(threads: int) -> dict:
    """The host the CPU baseline ran on: logical CPUs, threads used, lscpu's
    model name, sockets and cores per socket."""
    import subprocess
    info = {"cpu_count": os.cpu_count(), "threads": threads}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            key, _, val = line.partition(":")
            if key.strip() in ("Model name", "Socket(s)", "Core(s) per socket", "Thread(s) per core"):
                info[key.strip()] = val.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    return info


def cpu_baseline(torch, n_tokens: int) -> dict:
    """Reference-equivalent path on the host, fp32: the oracle Llama (HF layer
    math) with every layer under torch.utils.checkpoint(use_reentrant=False,
    debug=True) as the reference wrapper calls it, and with debug=False (the
    stock number).  `value` is a bounded sample of the metric's TinyLlama
    workload; beside it BASELINE config 1 (the whole debug model step) and
    config 2 (the memory-bound chain, op-level) on the same cores."""
    import torch.nn.functional as Fn
    from oracle.torch_llama import OracleLlama, rmsnorm, rope
    cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    prev = torch.get_num_threads()
    torch.set_num_threads(cores)

    def model_step(orc, ids, debug: bool) -> float:
        t0 = time.perf_counter()
        _, loss = orc.forward(ids, ids, checkpoint=True, debug=debug)
        loss.backward()
        return time.perf_counter() - t0

    try:
        c = TINYLLAMA
        orc = OracleLlama(vocab=c["vocab"], hidden=c["hidden"], n_layers=c["layers"], n_heads=c["heads"],
                          n_kv=c["kv"], ffn=c["ffn"], theta=c["theta"])
        ids = torch.randint(0, c["vocab"], (1, n_tokens), generator=torch.Generator().manual_seed(2000))
        model_step(orc, ids[:, :16], True)  # one-time initialisation outside the timed sample
        dt = model_step(orc, ids, True)
        dt_nd = model_step(orc, ids, False)
        del orc
        # config 1: the 2-layer debug model, batch 2 x 128 (median of 3 steps)
        tiny = OracleLlama(vocab=1024, hidden=256, n_layers=2, n_heads=8, n_kv=4, ffn=688, theta=10000.0)
        ids1 = torch.randint(0, 1024, (2, 128), generator=torch.Generator().manual_seed(2000))
        c1 = {d: sorted(model_step(tiny, ids1, d) for _ in range(3))[1] for d in (True, False)}
        # config 2: RMSNorm -> RoPE (32 x 128) + residual, SwiGLU [4096, 14336];
        # forward under the checkpoint (recomputed in backward) + backward
        sh = CHAIN_CFG2
        T, H, Fd, nr, hd = sh["tokens"], sh["hidden"], sh["ffn"], sh["rope_heads"], sh["head_dim"]
        gen = [torch.Generator().manual_seed(k) for k in range(1, 6)]
        x = torch.randn(1, T, H, generator=gen[0]).requires_grad_(True)
        wn = (1 + 0.02 * torch.randn(H, generator=gen[1])).requires_grad_(True)
        gt = torch.randn(1, T, Fd, generator=gen[2]).requires_grad_(True)
        ut = torch.randn(1, T, Fd, generator=gen[3]).requires_grad_(True)
        dyc = torch.randn(1, T, H, generator=gen[4])
        dpc = torch.randn(1, T, Fd, generator=gen[4])
        inv = 1.0 / (sh["theta"] ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd))
        ang = torch.arange(T, dtype=torch.float32)[:, None] * inv[None, :]
        ang = torch.cat((ang, ang), dim=-1)[None]
        cos, sin = ang.cos(), ang.sin()

        def chain(x_, g_, u_):
            y = rmsnorm(x_, wn, 1e-5)
            q = y.view(1, T, nr, hd).transpose(1, 2)
            qr, _ = rope(q, q, cos, sin)
            return qr.transpose(1, 2).reshape(1, T, H) + x_, Fn.silu(g_) * u_

        def chain_step(debug: bool) -> float:
            t0 = time.perf_counter()
            o1, o2 = torch.utils.checkpoint.checkpoint(chain, x, gt, ut, use_reentrant=False, debug=debug)
            torch.autograd.backward((o1, o2), (dyc, dpc))
            return time.perf_counter() - t0

        chain_step(True)  # one-time allocation outside the timed runs
        runs = {True: [], False: []}
        for _ in range(3):
            for d in (True, False):
                runs[d].append(chain_step(d))
        c2 = {d: sorted(v)[1] for d, v in runs.items()}
    finally:
        torch.set_num_threads(prev)
    return {"value": round(n_tokens / dt, 2), "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"1 fwd+bwd of the full 22-layer TinyLlama-1.1B-shaped model on 1 x {n_tokens} "
                      f"tokens, fp32, oracle/torch_llama.py layers under torch.utils.checkpoint("
                      f"use_reentrant=False, debug=True) as the reference wrapper calls it; "
                      f"{dt:.1f} s on {cores} threads",
            "debug_false": {"value": round(n_tokens / dt_nd, 2), "unit": "tokens/s",
                            "note": "same sample, torch.utils.checkpoint(debug=False)"},
            "config1": {"debug_true_tokens_per_s": round(256 / c1[True], 1),
                        "debug_false_tokens_per_s": round(256 / c1[False], 1),
                        "sample": "BASELINE config 1: the 2-layer debug model (hidden 256, 8 heads, "
                                  "4 KV heads, ffn 688, vocab 1024), one fwd+bwd of 2 x 128 tokens, "
                                  "median of 3"},
            "config2_chain": {"debug_true_ms": round(c2[True] * 1e3, 1),
                              "debug_false_ms": round(c2[False] * 1e3, 1),
                              "tokens_per_s": round(T / c2[True], 1),
                              "sample": "BASELINE config 2 op-level chain, fp32: RMSNorm, RoPE on "
                                        "32 x 128, residual add, SwiGLU [4096, 14336], forward under "
                                        "the checkpoint + recompute + backward (median of 3, interleaved)"},
            "host": host_info(cores)}


def main() -> int:
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (TP = PP = DP = 1); "
              "run it with --gpus 1", file=sys.stderr)
        return 2
    import torch

    from femtotron_amd import gemm_tuning
    if args.tune_gemms:
        gemm_tuning.tune(workloads=(args.workload,), path=args.tune_gemms, log=log)
        print(json.dumps({"tuned_gemms": args.tune_gemms}), flush=True)
        return 0
    tuned = False if args.no_tuned_gemms else gemm_tuning.use_tuned_gemms()
    log(f"library GEMMs: {'shipped TunableOp solutions' if tuned else 'default heuristics'}")
    from femtotron_amd import projections
    if args.tune_gemm_dispatch:
        wls = {name: (w["batch"] * w["seq"], w["hidden"], w["hidden"], w["kv"] * w["hidden"] // w["heads"],
                      w["ffn"], w["hidden"] // w["heads"], w["seq"]) for name, (w, _, _) in WORKLOADS.items()}
        path = projections.measure_dispatch(wls, log=log)
        print(json.dumps({"gemm_dispatch": str(path)}), flush=True)
        return 0
    projections.set_gemm_policy(args.gemm)
    from femtotron_amd.fused_layer import set_wgrad_side_stream
    set_wgrad_side_stream(args.wgrad_stream == "side")

    if args.profile_kernel:
        print(json.dumps(profile_kernel(torch, args.profile_kernel, WORKLOADS[args.workload][0])),
              flush=True)
        return 0

    from femtotron_amd import (dispatch_counts, fuse_attention, fuse_boundary_ops, fused_checkpoint,
                               pack_layer_weights, reset_dispatch_counts)
    from femtotron_amd.boundary_ops import unfuse_boundary_ops
    from femtotron_amd.fused_attention import (attention_dispatch_counts, reset_attention_dispatch_counts,
                                               unfuse_attention)
    from femtotron_amd.model import build_llama_model, init_llama_weights_
    from femtotron_amd.scripts.presets import get_ac_policy
    from femtotron_amd.training import apply_activation_checkpointing, remove_activation_checkpointing

    assert torch.cuda.is_available(), "bench.py needs a HIP device"
    c, model_name, cfg_name = WORKLOADS[args.workload]
    c = dict(c, layers=args.layers or c["layers"])
    L = c["layers"]
    B, S = c["batch"], c["seq"]
    T = B * S
    log(f"building {model_name}-shaped model ({L} layers), bf16, weights N(0, 0.02)")
    model = build_llama_model(llama_config(c, L))
    model = init_llama_weights_(model, device="cuda", dtype=torch.bfloat16, generator_device="cuda")
    packed_groups = pack_layer_weights(model)  # q/k/v and gate/up as row views of one buffer
    boundary = fuse_boundary_ops(model) if not args.stock_boundary else 0  # embedding, final norm
    # selective AC leaves attention outside the checkpoints: run it on the kernels too
    attn_fused = fuse_attention(model) if args.ac == "selective" and not args.stock_attention else 0
    policy = get_ac_policy(PRESETS[args.ac])
    apply_activation_checkpointing(model, policy, checkpoint_fn=fused_checkpoint)
    ids = torch.randint(0, c["vocab"], (B, S), generator=torch.Generator().manual_seed(2000)).cuda()

    reset_dispatch_counts()
    reset_attention_dispatch_counts()
    projections.reset_gemm_dispatch_counts()
    log(f"fused path ({args.ac} AC): {args.warmup} warm-up + {args.steps} timed steps")
    fused_head = not args.stock_loss_head
    sec = time_steps(torch, model, ids, args.steps, args.warmup, materialize_logits=not fused_head)
    counts = dispatch_counts()
    # selective: 2 norms + 1 MLP per layer, + the final norm unless fuse_boundary_ops took it
    calls_per_step = L if args.ac == "full" else 3 * L + (0 if boundary else 1)
    assert counts["fallback"] == 0 and counts["fused"] == calls_per_step * (args.steps + args.warmup), counts
    if attn_fused:
        acounts = attention_dispatch_counts()
        assert acounts == {"fused": L * (args.steps + args.warmup), "fallback": 0}, acounts
    tok_s = T / sec
    gemm_counts = projections.gemm_dispatch_counts()
    n_steps = args.steps + args.warmup
    gemm_counts = {k: v // n_steps for k, v in gemm_counts.items()}
    log(f"fused: {sec * 1e3:.2f} ms/step, {tok_s:.0f} tokens/s; projection GEMMs per step: "
        f"{gemm_counts['hand']} hand-written, {gemm_counts['library']} library")
    auto_step = None
    if args.gemm == "hand" and not args.no_auto_gemm_step:
        # The same step with the forward (NT) GEMMs the measured table gives the
        # library on it: a reported comparison, not the metric.
        projections.set_gemm_policy("auto")
        projections.reset_gemm_dispatch_counts()
        asec = time_steps(torch, model, ids, args.steps, args.warmup, materialize_logits=not fused_head)
        acounts_g = {k: v // n_steps for k, v in projections.gemm_dispatch_counts().items()}
        projections.set_gemm_policy("hand")
        auto_step = {"tokens_per_s": round(T / asec, 1), "ms_per_step": round(asec * 1e3, 3),
                     "projection_gemms_per_step": acounts_g,
                     "note": "the same step under --gemm auto (the library where the table measured it "
                             "faster), timed after the metric's steps"}
        log(f"same step, --gemm auto: {asec * 1e3:.2f} ms/step, {T / asec:.0f} tokens/s")

    log("per-kernel HIP-event timings at the step's shapes")
    rows, mfma = kernel_table(torch, c, args.kernel_iters, args.ac, boundary=bool(boundary),
                              fused_attention=bool(attn_fused))
    for r in rows:
        r["ms_per_step"] = round(r["event_ms_per_launch"] * r["launches_per_step"], 4)
    for r in mfma:
        r["ms_per_step"] = round(r["ms_per_launch"] * r["launches_per_step"], 4)
    timing = (f"mean of {args.kernel_iters} back-to-back launches alone at the step's shape, HIP events "
              "on the launch stream, after ~40 ms of launches that let the clock settle (fused_kernels_hbm rows: ms_per_launch is the kernels' own execution "
              "time from torch.profiler device timestamps, event_ms_per_launch the HIP-event mean)")
    dom = max(rows, key=lambda r: r["ms_per_step"])
    ev_gbs = dom["bytes_per_launch"] / (dom["event_ms_per_launch"] * 1e-3) / 1e9
    roofline_hbm = {"bound": "hbm", "kernel": dom["kernel"], "achieved": round(ev_gbs, 1),
                    "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(ev_gbs / HBM_PEAK_GBS, 4),
                    "traffic": measured_traffic(dom["kernel"]) if args.workload == "tinyllama" else None,
                    "bytes_per_launch": dom["bytes_per_launch"],
                    "us_per_launch": round(dom["event_ms_per_launch"] * 1e3, 2), "duration": timing,
                    "kernel_only_frac": dom["frac"]}
    # The dominant kernel of this build: the hand-written kernel (fused HBM,
    # attention or projection GEMM on fh_gemm_bf16) with the most time per step.
    own = [r for r in mfma if not r.get("path", "fh").startswith("library")]
    dom_m = max(own, key=lambda r: r["ms_per_step"]) if own else None
    if dom_m is not None and dom_m["ms_per_step"] > dom["ms_per_step"]:
        roofline = {"bound": "mfma", "kernel": dom_m["kernel"], "achieved": dom_m["achieved_tflops"],
                    "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": dom_m["frac"],
                    "traffic": measured_traffic(dom_m["kernel"]) if args.workload == "tinyllama" else None,
                    "flop_per_launch": dom_m["flop_per_launch"],
                    "us_per_launch": round(dom_m["ms_per_launch"] * 1e3, 2), "duration": timing}
    else:
        roofline = roofline_hbm

    def use(fused: bool):
        remove_activation_checkpointing(model)
        if boundary:
            (fuse_boundary_ops if fused else unfuse_boundary_ops)(model)
        if attn_fused:
            (fuse_attention if fused else unfuse_attention)(model)
        if fused:
            apply_activation_checkpointing(model, policy, checkpoint_fn=fused_checkpoint)
        else:
            apply_activation_checkpointing(model, policy)  # default checkpoint_fn = torch's
        torch.cuda.empty_cache()

    ref = None
    if args.reference_steps > 0:
        log("reference path on the same GPU: HF layers under torch.utils.checkpoint(debug=True)")
        use(False)
        rsec = time_steps(torch, model, ids, args.reference_steps, 1)
        ref = {"tokens_per_s": round(T / rsec, 1), "ms_per_step": round(rsec * 1e3, 2),
               "speedup_fused_vs_reference": round(rsec / sec, 2),
               "checkpoint": "torch.utils.checkpoint(use_reentrant=False, debug=True), as the reference's "
                             "wrapper calls it (femtotron/training/activation_ckpt.py:84)"}
        log(f"reference: {rsec * 1e3:.1f} ms/step")
        # the stock number: the same path with the checkpoint's debug traces off
        from torch.utils.checkpoint import checkpoint as torch_checkpoint

        def checkpoint_no_debug(fn, *a, **k):
            k["debug"] = False
            return torch_checkpoint(fn, *a, **k)

        remove_activation_checkpointing(model)
        apply_activation_checkpointing(model, policy, checkpoint_fn=checkpoint_no_debug)
        rsec_nd = time_steps(torch, model, ids, args.reference_steps, 1)
        ref["debug_false"] = {"tokens_per_s": round(T / rsec_nd, 1), "ms_per_step": round(rsec_nd * 1e3, 2),
                              "speedup_fused_vs_reference": round(rsec_nd / sec, 2)}
        log(f"reference, debug=False: {rsec_nd * 1e3:.1f} ms/step")
    # Activation memory, measured back to back for both paths in the same
    # allocator state (each after one step of its own to allocate gradients).
    use(True)
    act_fused = activation_bytes_per_token(torch, model, ids, materialize_logits=not fused_head)
    if ref is not None:
        use(False)
        ref["activation_bytes_per_token"] = round(activation_bytes_per_token(torch, model, ids), 1)
    optimizer = None
    if not args.no_optimizer:
        log("mixed-precision AdamW step: fused vs the reference's sequence")
        optimizer = optimizer_timing(torch, model, args.kernel_iters)
        log(f"optimizer: fused {optimizer['ms_per_step']:.2f} ms, reference "
            f"{optimizer['reference_ms_per_step']:.2f} ms")
    del model
    torch.cuda.empty_cache()

    chain = None
    if not args.no_chain:
        log("BASELINE config 2: the memory-bound chain op-level, MALL flushed before every launch")
        chain = {"shape": CHAIN_CFG2, "rows": chain_table(torch, CHAIN_CFG2, max(10, args.kernel_iters)),
                 "duration": "kernel execution time (torch.profiler device timestamps, the rocprofv3 kernel-trace "
                             "durations), median of one launch per session after a 512 MiB read that evicts the "
                             "MALL; event_ms_per_launch: HIP events around the same launch"}
        torch.cuda.empty_cache()

    cpu = None
    if args.cpu_sample_tokens > 0 and args.workload == "tinyllama":
        log(f"cpu baseline: {args.cpu_sample_tokens} tokens on the host")
        cpu = cpu_baseline(torch, args.cpu_sample_tokens)

    step_flops = None
    if args.ac == "full":
        fl = step_flops_per_token(c)
        step_flops = {"model_gflop_per_token": round(fl["model"] / 1e9, 3),
                      "hardware_gflop_per_token": round(fl["hardware"] / 1e9, 3),
                      "mfu": round(fl["model"] * tok_s / (MFMA_BF16_PEAK_TFLOPS * 1e12), 4),
                      "hfu": round(fl["hardware"] * tok_s / (MFMA_BF16_PEAK_TFLOPS * 1e12), 4),
                      "note": "layer forward (projection GEMMs + causal attention 2 Hq S per token) x3 "
                              "(model) or x4 less the down projection (hardware: the recompute stops at "
                              "SwiGLU), lm_head x3, against 2.5 PFLOP/s dense bf16"}

    metric = METRIC if args.workload == "tinyllama" else f"ckpt'd fwd+bwd tokens/s @1 GPU ({model_name})"
    out = {
        "metric": metric, "value": round(tok_s, 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(sec * 1e3, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (token ids uniform over the vocab, CPU Generator(2000); random-init "
                "weights N(0, 0.02))",
        "config": {"workload": f"{model_name}-shaped checkpointed fwd+bwd ({cfg_name})",
                   "layers": L, "hidden": c["hidden"], "heads": c["heads"],
                   "kv_heads": c["kv"], "ffn": c["ffn"], "vocab": c["vocab"], "micro_batch": B,
                   "seq_len": S, "tokens_per_step": T,
                   "activation_checkpointing": "every layer" if args.ac == "full"
                   else "selective: every LlamaMLP and LlamaRMSNorm; attention outside the "
                        + ("checkpoints on the fused kernels (fuse_attention)" if attn_fused
                           else "checkpoints as HF's LlamaAttention"),
                   "parallelism": "single GPU (TP=PP=DP=1)"},
        "roofline": roofline,
        "roofline_hbm": roofline_hbm,
        "step_flops": step_flops,
        "fused_kernels_hbm": rows,
        "op_level_chain_cfg2": chain,
        "mfma_kernels": mfma,
        "gemms": {"policy": args.gemm,
                  "projection_gemms_per_step": gemm_counts,
                  "step_under_auto_policy": auto_step,
                  "hand_written": "fh_gemm_bf16 (femtotron_amd/csrc/fh_gemm.hip)",
                  "library": ("hipBLASLt/rocBLAS, TunableOp solutions from femtotron_amd/tuned/"
                              "tunableop_gfx950.csv" if tuned else "hipBLASLt default heuristics"),
                  "table": "femtotron_amd/tuned/gemm_dispatch_gfx950.json",
                  "weight_gradients": ("in series with the input-gradient chain" if args.wgrad_stream == "serial"
                                       else "side stream")},
        "weights": f"q/k/v and gate/up packed contiguously ({packed_groups} groups)",
        "boundary_ops": ("fused embedding (deterministic scatter-add backward) and final RMSNorm"
                         if boundary else "reference nn.Embedding and LlamaRMSNorm"),
        "loss_head": ("fused lm_head + chunked cross-entropy (materialize_logits=False)" if fused_head
                      else "reference: materialised logits, fp32 cross-entropy"),
        "activation_bytes_per_token": round(act_fused, 1),
        "reference_gpu": ref,
        "optimizer_step": optimizer,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
