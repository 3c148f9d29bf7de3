// Causal-LM cross-entropy over a chunk of logits rows, forward and gradient in
// one pass, in place.
//
// Reference: femtotron/model/base.py:24-31 and femtotron/model/llama.py:104-111,
//   F.cross_entropy(logits.float().view(-1, V), labels.view(-1), ignore_index=-100)
// (mean over the non-ignored rows) after the next-token shift; its autograd
// gradient is (softmax(x) - onehot(label)) / n_valid in fp32, rounded to the
// logits' dtype by the backward of .float().
//
// One workgroup of 1024 threads per row: thread t owns the 8-element chunks
// (i*1024 + t)*8, i < NV, so every load instruction of a wave covers one
// contiguous 1 KiB (bf16) span and the row stays in registers between the
// reductions and the gradient; the logits are read from HBM once and written
// once.  Row max and sum of exponentials: wave DPP reductions, then a fixed-order
// combine of the 16 waves through LDS (deterministic).
#include <math.h>

#include <type_traits>

#include "fh_common.hpp"

namespace fh {
namespace {

constexpr int kCeThreads = 1024;
constexpr float kLog2eF = 1.4426950408889634f;
constexpr float kLn2F = 0.6931471805599453f;
constexpr int kCeWaves = kCeThreads / kWave;

// Max and sum over the workgroup (every thread gets the result).
__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  const int wave = threadIdx.x >> 6;
  __syncthreads();  // red may still be read by the previous reduction
  if ((threadIdx.x & (kWave - 1)) == 0) red[wave] = v;
  __syncthreads();
  float m = red[0];
#pragma unroll
  for (int w = 1; w < kCeWaves; ++w) m = fmaxf(m, red[w]);
  return m;
}

__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int wave = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & (kWave - 1)) == 0) red[wave] = v;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int w = 0; w < kCeWaves; ++w) s += red[w];
  return s;
}

template <typename T, int NV>
__global__ __launch_bounds__(kCeThreads) void k_ce_rows(T* __restrict__ logits, int64_t ld,
                                                        const int64_t* __restrict__ labels,
                                                        int64_t vocab, int64_t ignore_index,
                                                        const float* __restrict__ inv_count,
                                                        float* __restrict__ loss_rows) {
  using Raw = typename Elem<T>::Raw;
  __shared__ float red[kCeWaves];
  __shared__ float x_label;
  const int64_t row = blockIdx.x;
  T* x = logits + row * ld;
  const int64_t label = labels[row];
  const bool ignored = label == ignore_index;
  // A label outside [0, vocab) (torch raises there) marks the row NaN; it is
  // never used to address memory.
  const bool valid = !ignored && label >= 0 && label < vocab;
  const bool bad = !ignored && !valid;

  Raw r[NV];
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t c = (static_cast<int64_t>(i) * kCeThreads + threadIdx.x) * 8;
    if (c < vocab) {
      r[i] = Elem<T>::ldraw(x + c);
      float v[8];
      Elem<T>::unpack(r[i], v);
#pragma unroll
      for (int j = 0; j < 8; ++j) m = fmaxf(m, v[j]);
    }
  }
  if (threadIdx.x == 0) x_label = valid ? Elem<T>::ld1(x + label) : 0.f;
  // Exponentials in the log2 domain on v_exp_f32 / v_log_f32 (~1 ulp each):
  // e^(x - m) = 2^(x*log2e - m*log2e), one FMA and one transcendental per term.
  const float m2 = block_max(m, red) * kLog2eF;
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t c = (static_cast<int64_t>(i) * kCeThreads + threadIdx.x) * 8;
    if (c < vocab) {
      float v[8];
      Elem<T>::unpack(r[i], v);
#pragma unroll
      for (int j = 0; j < 8; ++j) s += __builtin_amdgcn_exp2f(fmaf(v[j], kLog2eF, -m2));
    }
  }
  s = block_sum(s, red);  // its barriers also publish x_label
  const float lse2 = m2 + __builtin_amdgcn_logf(s);  // log2-sum-exp2 in log2 units
  if (threadIdx.x == 0) loss_rows[row] = valid ? lse2 * kLn2F - x_label : (bad ? NAN : 0.f);
  const float scale = valid ? *inv_count : (bad ? NAN : 0.f);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t c = (static_cast<int64_t>(i) * kCeThreads + threadIdx.x) * 8;
    if (c < vocab) {
      float v[8];
      Elem<T>::unpack(r[i], v);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float p = __builtin_amdgcn_exp2f(fmaf(v[j], kLog2eF, -lse2));
        v[j] = (c + j == label ? p - 1.f : p) * scale;
      }
      Elem<T>::store8(x + c, v);
    }
  }
}

// Vocabularies above 8 chunks per thread (65,536) do not fit the registers of
// a 1024-thread workgroup; they stream the row twice instead: an online
// max / sum-of-exponentials pass, then the gradient pass (1.5x the traffic).
template <typename T>
__global__ __launch_bounds__(kCeThreads) void k_ce_rows_stream(T* __restrict__ logits, int64_t ld,
                                                               const int64_t* __restrict__ labels,
                                                               int64_t vocab, int64_t ignore_index,
                                                               const float* __restrict__ inv_count,
                                                               float* __restrict__ loss_rows) {
  __shared__ float red[kCeWaves];
  __shared__ float x_label;
  const int64_t row = blockIdx.x;
  T* x = logits + row * ld;
  const int64_t label = labels[row];
  const bool ignored = label == ignore_index;
  const bool valid = !ignored && label >= 0 && label < vocab;
  const bool bad = !ignored && !valid;
  if (threadIdx.x == 0) x_label = valid ? Elem<T>::ld1(x + label) : 0.f;
  const int64_t step = static_cast<int64_t>(kCeThreads) * 8;
  float m2 = -INFINITY, s = 0.f;  // running max (log2 units) and sum of 2^(x log2e - m2)
  for (int64_t c = static_cast<int64_t>(threadIdx.x) * 8; c < vocab; c += step) {
    float v[8];
    Elem<T>::load8(x + c, v);
    float cm = v[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) cm = fmaxf(cm, v[j]);
    const float nm2 = fmaxf(m2, cm * kLog2eF);
    s *= __builtin_amdgcn_exp2f(m2 - nm2);
    m2 = nm2;
#pragma unroll
    for (int j = 0; j < 8; ++j) s += __builtin_amdgcn_exp2f(fmaf(v[j], kLog2eF, -m2));
  }
  const float bm2 = block_max(m2, red);
  s = block_sum(m2 == -INFINITY ? 0.f : s * __builtin_amdgcn_exp2f(m2 - bm2), red);
  const float lse2 = bm2 + __builtin_amdgcn_logf(s);
  if (threadIdx.x == 0) loss_rows[row] = valid ? lse2 * kLn2F - x_label : (bad ? NAN : 0.f);
  const float scale = valid ? *inv_count : (bad ? NAN : 0.f);
  for (int64_t c = static_cast<int64_t>(threadIdx.x) * 8; c < vocab; c += step) {
    float v[8];
    Elem<T>::load8(x + c, v);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float p = __builtin_amdgcn_exp2f(fmaf(v[j], kLog2eF, -lse2));
      v[j] = (c + j == label ? p - 1.f : p) * scale;
    }
    Elem<T>::store8(x + c, v);
  }
}

// Chunks of 8 per thread held in registers (0 = stream the row).
template <typename F>
int dispatch_ce_nv(int64_t vocab, F&& f) {
  const int64_t per = static_cast<int64_t>(kCeThreads) * 8;
  if (vocab <= per) return f(std::integral_constant<int, 1>{});
  if (vocab <= 2 * per) return f(std::integral_constant<int, 2>{});
  if (vocab <= 4 * per) return f(std::integral_constant<int, 4>{});
  if (vocab <= 8 * per) return f(std::integral_constant<int, 8>{});
  return f(std::integral_constant<int, 0>{});
}

}  // namespace
}  // namespace fh

using namespace fh;

extern "C" int fh_ce_fwd_bwd(fh_dtype dt, void* logits, int64_t ld, const int64_t* labels,
                             int64_t rows, int64_t vocab, int64_t ignore_index,
                             const float* inv_count, float* loss_rows, hipStream_t stream) {
  FH_REQUIRE(dt == FH_BF16 || dt == FH_F32, "ce_fwd_bwd: dtype must be FH_BF16 or FH_F32");
  FH_REQUIRE(rows >= 0, "ce_fwd_bwd: rows must be >= 0");
  FH_REQUIRE(vocab > 0 && vocab % 8 == 0 && vocab <= 0x7fffffff,
             "ce_fwd_bwd: vocab must be a positive multiple of 8");
  FH_REQUIRE(ld >= vocab && ld % 8 == 0, "ce_fwd_bwd: ld must be >= vocab and a multiple of 8");
  FH_REQUIRE(rows <= 0x7fffffff, "ce_fwd_bwd: too many rows");
  if (rows == 0) return FH_OK;
  FH_REQUIRE(logits && labels && inv_count && loss_rows, "ce_fwd_bwd: null pointer");
  FH_REQUIRE(aligned16(logits), "ce_fwd_bwd: logits must be 16-byte aligned");
  auto go = [&](auto tag, auto nv) {
    using T = decltype(tag);
    constexpr int NV = decltype(nv)::value;
    const dim3 grid(static_cast<unsigned>(rows));
    if constexpr (NV == 0)
      hipLaunchKernelGGL((k_ce_rows_stream<T>), grid, dim3(kCeThreads), 0, stream,
                         static_cast<T*>(logits), ld, labels, vocab, ignore_index, inv_count, loss_rows);
    else
      hipLaunchKernelGGL((k_ce_rows<T, NV>), grid, dim3(kCeThreads), 0, stream,
                         static_cast<T*>(logits), ld, labels, vocab, ignore_index, inv_count, loss_rows);
    return 0;
  };
  dispatch_ce_nv(vocab, [&](auto nv) {
    return dt == FH_BF16 ? go(uint16_t{}, nv) : go(float{}, nv);
  });
  return check_launch("fh_ce_fwd_bwd");
}
