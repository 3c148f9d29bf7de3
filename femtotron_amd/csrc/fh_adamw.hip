// Mixed-precision AdamW step over many tensors: the global gradient norm and
// clipping coefficient (a streaming sum-of-squares pass and two small
// deterministic folds), then one fused update pass.
//
// Reference (femtotron/training/mixed_precision_manager.py:318-331 step()):
//   master.grad = param.grad.float()                              (:190-249)
//   ClipGradNorm: total = sqrt(sum over grads of sum(g^2)),
//     coef = clamp(max_norm / (total + 1e-6), max=1), g *= coef   (grad_transform.py:13-63)
//   torch.optim.AdamW on the fp32 masters (femtotron/scripts/train.py:264-276; per-group
//     weight decay from optimizer.py:4-45), i.e. per element
//     p *= 1 - lr*wd;  m = lerp(m, g, 1-b1);  v = v*b2 + (1-b2)*g*g
//     p -= (lr/bc1) * m / (sqrt(v)/sqrt(bc2) + eps)
//   param.copy_(master)                                           (param_group.py:82-87)
// Each element is read once (bf16 grad, fp32 master, m, v) and written once
// (master, m, v, bf16 param): 28 bytes per parameter.
//
// Tensor table (device memory, built by the caller): entry i describes tensor i.
#include <math.h>

#include "fh_common.hpp"

namespace fh {
namespace {

constexpr int kAdamThreads = 256;
constexpr int64_t kAdamChunk = kAdamThreads * 8;  // elements per block and pass

// Block -> tensor: chunk_start[i] = first chunk of tensor i (prefix sums,
// chunk_start[n] = total chunks); binary search, uniform per block.
__device__ __forceinline__ int find_tensor(const int64_t* chunk_start, int n, int64_t chunk) {
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (chunk_start[mid] <= chunk) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

// Pass 1: per-block fp32 sum of squares of the (model-dtype) gradients over
// kSqChunks consecutive chunks.  When they all lie in one tensor (every block
// of a large tensor) the loads are issued together; a block that crosses a
// tensor boundary walks its chunks one by one.
constexpr int kSqChunks = 8;

template <typename G>
__global__ __launch_bounds__(kAdamThreads) void k_grad_sq(const FhAdamTensor* __restrict__ tab,
                                                          const int64_t* __restrict__ chunk_start,
                                                          int n, int64_t total, float* __restrict__ part) {
  __shared__ float red[kAdamThreads / kWave];
  const int64_t c0 = static_cast<int64_t>(blockIdx.x) * kSqChunks;
  const int64_t c1 = c0 + kSqChunks < total ? c0 + kSqChunks : total;
  int ti = find_tensor(chunk_start, n, c0);
  float s = 0.f;
  if (c1 <= chunk_start[ti + 1] &&
      (c1 - chunk_start[ti]) * kAdamChunk <= tab[ti].numel) {  // whole chunks of one tensor
    const G* gp = static_cast<const G*>(tab[ti].grad) + (c0 - chunk_start[ti]) * kAdamChunk + threadIdx.x * 8;
    if (c1 - c0 == kSqChunks) {
      float g[kSqChunks][8];
#pragma unroll
      for (int u = 0; u < kSqChunks; ++u) Elem<G>::load8(gp + u * kAdamChunk, g[u]);
#pragma unroll
      for (int u = 0; u < kSqChunks; ++u)
#pragma unroll
        for (int j = 0; j < 8; ++j) s = fmaf(g[u][j], g[u][j], s);
    } else {
      for (int64_t c = c0; c < c1; ++c, gp += kAdamChunk) {
        float g[8];
        Elem<G>::load8(gp, g);
#pragma unroll
        for (int j = 0; j < 8; ++j) s = fmaf(g[j], g[j], s);
      }
    }
  } else {
    for (int64_t c = c0; c < c1; ++c) {
      while (chunk_start[ti + 1] <= c) ++ti;  // chunk_start[n] = total > c ends the walk
      const FhAdamTensor t = tab[ti];
      const G* gp = static_cast<const G*>(t.grad);
      const int64_t i0 = (c - chunk_start[ti]) * kAdamChunk + threadIdx.x * 8;
      if (i0 + 8 <= t.numel) {
        float g[8];
        Elem<G>::load8(gp + i0, g);
#pragma unroll
        for (int j = 0; j < 8; ++j) s = fmaf(g[j], g[j], s);
      } else {
        for (int64_t i = i0; i < t.numel; ++i) {
          const float g = Elem<G>::ld1(gp + i);
          s = fmaf(g, g, s);
        }
      }
    }
  }
  s = wave_sum(s);
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    float b = 0.f;
#pragma unroll
    for (int w = 0; w < kAdamThreads / kWave; ++w) b += red[w];
    part[blockIdx.x] = b;
  }
}

// Pass 2a: kFoldBlocks blocks each sum one contiguous slice of the partials.
constexpr int kFoldBlocks = 256;

__global__ __launch_bounds__(kAdamThreads) void k_fold_parts(const float* __restrict__ part, int64_t nparts,
                                                             float* __restrict__ out) {
  __shared__ float red[kAdamThreads / kWave];
  const int64_t span = (nparts + kFoldBlocks - 1) / kFoldBlocks;
  const int64_t lo = blockIdx.x * span;
  const int64_t hi = lo + span < nparts ? lo + span : nparts;
  float s = 0.f;
  for (int64_t i = lo + threadIdx.x; i < hi; i += kAdamThreads) s += part[i];
  s = wave_sum(s);
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    float b = 0.f;
#pragma unroll
    for (int w = 0; w < kAdamThreads / kWave; ++w) b += red[w];
    out[blockIdx.x] = b;
  }
}

// Pass 2b: one wave folds the kFoldBlocks sums in a fixed order and writes the
// clipping coefficient and the total norm (coef = 1 when max_norm <= 0).
__global__ __launch_bounds__(kWave) void k_clip_coef(const float* __restrict__ folded, float max_norm,
                                                     float* __restrict__ out) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kFoldBlocks / kWave; ++i) s += folded[i * kWave + threadIdx.x];
  s = wave_sum(s);
  if (threadIdx.x == 0) {
    const float norm = sqrtf(s);
    out[0] = max_norm > 0.f ? fminf(max_norm / (norm + 1e-6f), 1.f) : 1.f;
    out[1] = norm;
  }
}

// Pass 3: the update.  G = gradient / parameter dtype (bf16 or fp32).
template <typename G>
__global__ __launch_bounds__(kAdamThreads) void k_adamw(const FhAdamTensor* __restrict__ tab,
                                                        const int64_t* __restrict__ chunk_start,
                                                        int n, const float* __restrict__ coef_p,
                                                        FhAdamHyper hp) {
  const int64_t chunk = blockIdx.x;
  const int ti = find_tensor(chunk_start, n, chunk);
  const FhAdamTensor t = tab[ti];
  const int64_t i = (chunk - chunk_start[ti]) * kAdamChunk + threadIdx.x * 8;
  if (i >= t.numel) return;
  const float coef = *coef_p;
  auto update = [&](float g, float& p, float& m, float& v) {
    const float gj = g * coef;
    p *= t.decay;                                               // mul_(1 - lr*wd)
    m = m + hp.one_minus_beta1 * (gj - m);                      // lerp_(g, 1 - beta1)
    v = __fmul_rn(v, hp.beta2) + hp.one_minus_beta2 * gj * gj;  // mul_(beta2).addcmul_(g, g, 1 - beta2)
    const float denom = sqrtf(v) / t.bias_correction2_sqrt + hp.eps;
    p = p - t.step_size * (m / denom);                          // addcdiv_(m, denom, -step_size)
  };
  if (i + 8 <= t.numel) {
    float g[8], p[8], m[8], v[8];
    Elem<G>::load8(static_cast<const G*>(t.grad) + i, g);
    Elem<float>::load8(t.master + i, p);
    Elem<float>::load8(t.exp_avg + i, m);
    Elem<float>::load8(t.exp_avg_sq + i, v);
#pragma unroll
    for (int j = 0; j < 8; ++j) update(g[j], p[j], m[j], v[j]);
    Elem<float>::store8(t.master + i, p);
    Elem<float>::store8(t.exp_avg + i, m);
    Elem<float>::store8(t.exp_avg_sq + i, v);
    Elem<G>::store8(static_cast<G*>(t.param) + i, p);  // param.copy_(master)
  } else {
    for (int64_t e = i; e < t.numel; ++e) {
      float p = t.master[e], m = t.exp_avg[e], v = t.exp_avg_sq[e];
      update(Elem<G>::ld1(static_cast<const G*>(t.grad) + e), p, m, v);
      t.master[e] = p;
      t.exp_avg[e] = m;
      t.exp_avg_sq[e] = v;
      Elem<G>::st1(static_cast<G*>(t.param) + e, p);
    }
  }
}

}  // namespace
}  // namespace fh

using namespace fh;

// Workspace (floats): [0, total_chunks) pass-1 partials, then the clipping
// coefficient and the norm, then kFoldBlocks folded sums.
extern "C" size_t fh_adamw_workspace_size(int64_t total_chunks) {
  return total_chunks > 0 ? static_cast<size_t>(total_chunks + 2 + kFoldBlocks) * sizeof(float) : 0;
}

extern "C" int fh_adamw_step(fh_dtype dt, const FhAdamTensor* table, const int64_t* chunk_start,
                             int n_tensors, int64_t total_chunks, FhAdamHyper hyper,
                             float max_grad_norm, void* workspace, hipStream_t stream) {
  FH_REQUIRE(dt == FH_BF16 || dt == FH_F32, "adamw_step: dtype must be FH_BF16 or FH_F32");
  FH_REQUIRE(n_tensors >= 0 && total_chunks >= 0, "adamw_step: negative size");
  if (n_tensors == 0 || total_chunks == 0) return FH_OK;
  FH_REQUIRE(table && chunk_start && workspace, "adamw_step: null pointer");
  FH_REQUIRE(total_chunks <= 0x7fffffff, "adamw_step: too many chunks");
  float* part = static_cast<float*>(workspace);
  float* coef = part + total_chunks;  // coef, norm
  float* folded = coef + 2;
  const dim3 grid(static_cast<unsigned>(total_chunks));
  const int64_t nparts = (total_chunks + kSqChunks - 1) / kSqChunks;
  const dim3 sq_grid(static_cast<unsigned>(nparts));
  if (dt == FH_BF16) {
    hipLaunchKernelGGL(k_grad_sq<uint16_t>, sq_grid, dim3(kAdamThreads), 0, stream, table, chunk_start,
                       n_tensors, total_chunks, part);
  } else {
    hipLaunchKernelGGL(k_grad_sq<float>, sq_grid, dim3(kAdamThreads), 0, stream, table, chunk_start,
                       n_tensors, total_chunks, part);
  }
  hipLaunchKernelGGL(k_fold_parts, dim3(kFoldBlocks), dim3(kAdamThreads), 0, stream, part, nparts, folded);
  hipLaunchKernelGGL(k_clip_coef, dim3(1), dim3(kWave), 0, stream, folded, max_grad_norm, coef);
  if (dt == FH_BF16) {
    hipLaunchKernelGGL(k_adamw<uint16_t>, grid, dim3(kAdamThreads), 0, stream, table, chunk_start,
                       n_tensors, coef, hyper);
  } else {
    hipLaunchKernelGGL(k_adamw<float>, grid, dim3(kAdamThreads), 0, stream, table, chunk_start,
                       n_tensors, coef, hyper);
  }
  return check_launch("fh_adamw_step");
}
