// RMSNorm forward / residual-add + RMSNorm forward / RMSNorm backward.
//
// Reference arithmetic: LlamaRMSNorm.forward, transformers 5.15.0
// models/llama/modeling_llama.py:62-67, and the residual adds at :317/:323.
//
// Layout: one wave64 per row.  Lane l owns the 8-element chunks starting at
// columns (i*64 + l)*8, i < NV, so each load instruction of a wave covers one
// contiguous 1 KiB (bf16) span of the row; the row stays in registers between
// the reduction and the normalisation, so x is read from HBM exactly once.
#include "fh_common.hpp"

namespace fh {
namespace {

constexpr int kRowsPerBlock = 4;  // 4 waves = 256 threads

// Rows per wave kept in flight (FH_NORM_FWD_ROWS).  One row per wave, i.e.
// more waves, measured faster than two rows per wave at T=16384, H=2048
// (4.76 vs 4.39 TB/s).
#ifndef FH_NORM_FWD_ROWS
#define FH_NORM_FWD_ROWS 1
#endif
template <int NV>
struct FwdRows {
  static constexpr int R = NV <= 4 ? FH_NORM_FWD_ROWS : 1;
};

template <typename T, int NV, bool ADD>
__global__ __launch_bounds__(256) void k_rmsnorm_fwd(
    const T* __restrict__ x, const T* __restrict__ a, const T* __restrict__ w,
    T* __restrict__ h, T* __restrict__ y, float* __restrict__ rstd,
    int64_t rows, int cols, float eps) {
  constexpr int R = FwdRows<NV>::R;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6)) * R;
  if (row0 >= rows) return;  // uniform per wave

  float v[R][NV][8];
#pragma unroll
  for (int k = 0; k < R; ++k) {
    const int64_t base = (row0 + k) * cols;
    const bool ok = row0 + k < rows;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = (i * kWave + lane) * 8;
      if (ok && c < cols) {
        Elem<T>::load8(x + base + c, v[k][i]);
        if constexpr (ADD) {
          float b[8];
          Elem<T>::load8(a + base + c, b);
#pragma unroll
          for (int j = 0; j < 8; ++j) v[k][i][j] = Elem<T>::rnd(v[k][i][j] + b[j]);
          Elem<T>::store8(h + base + c, v[k][i]);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[k][i][j] = 0.f;
      }
    }
  }
#pragma unroll
  for (int k = 0; k < R; ++k) {
    if (row0 + k >= rows) break;  // uniform per wave
    const int64_t base = (row0 + k) * cols;
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) ss = fmaf(v[k][i][j], v[k][i][j], ss);
    ss = wave_sum(ss);
    const float r = rsqrtf(ss / static_cast<float>(cols) + eps);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = (i * kWave + lane) * 8;
      if (c < cols) {
        float wv[8], o[8];
        Elem<T>::load8(w + c, wv);
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = Elem<T>::rnd(wv[j] * Elem<T>::rnd(v[k][i][j] * r));
        Elem<T>::store8(y + base + c, o);
      }
    }
    if (rstd != nullptr && lane == 0) rstd[row0 + k] = r;
  }
}

// Backward.  Each wave walks row pairs (row0, row0 + S), (row0 + 2S, ...) with
// S = 4*gridDim.x, issuing all loads of a pair (x, dy and the residual
// gradient, kept packed until used) before the first reduction, and keeps its
// share of the weight gradient in registers; the 4 waves of a block are then
// summed in a fixed order through LDS into one fp32 partial row per block
// (deterministic), which k_reduce_cols folds into dw.
template <typename T, int NV, bool RES, bool HAVE_RSTD>
__global__ __launch_bounds__(256) void k_rmsnorm_bwd(
    const T* __restrict__ dy, const T* __restrict__ x, const T* __restrict__ w,
    const float* __restrict__ rstd, const T* __restrict__ dres,
    T* __restrict__ dx, float* __restrict__ part, int64_t rows, int cols,
    float eps) {
  using Raw = typename Elem<T>::Raw;
  constexpr int R = NV <= 4 ? 2 : 1;
  extern __shared__ float lds_acc[];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;

  float acc[NV][8];
#pragma unroll
  for (int i = 0; i < NV; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = 0.f;

  const float inv_cols = 1.f / static_cast<float>(cols);
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kRowsPerBlock;
  for (int64_t row0 = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + wave; row0 < rows;
       row0 += R * stride) {
    Raw xr[R][NV], gr[R][NV], rr[R][NV];
#pragma unroll
    for (int k = 0; k < R; ++k) {
      const int64_t row = row0 + k * stride;
      const int64_t base = row * cols;
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int c = (i * kWave + lane) * 8;
        if (row < rows && c < cols) {
          xr[k][i] = Elem<T>::ldraw(x + base + c);
          gr[k][i] = Elem<T>::ldraw(dy + base + c);
          if constexpr (RES) rr[k][i] = Elem<T>::ldraw(dres + base + c);
        }
      }
    }
#pragma unroll
    for (int k = 0; k < R; ++k) {
      const int64_t row = row0 + k * stride;
      if (row >= rows) break;  // uniform per wave
      const int64_t base = row * cols;
      float r;
      if constexpr (HAVE_RSTD) {
        r = rstd[row];
      } else {
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
          if ((i * kWave + lane) * 8 < cols) {
            float xv[8];
            Elem<T>::unpack(xr[k][i], xv);
#pragma unroll
            for (int j = 0; j < 8; ++j) ss = fmaf(xv[j], xv[j], ss);
          }
        }
        r = rsqrtf(wave_sum(ss) * inv_cols + eps);
      }
      // dn = to_dtype(dy*w) is the gradient arriving at the bf16 normalised
      // value; dot = mean(dn * n) over the row.
      float dot = 0.f;
      float dn[NV][8];
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int c = (i * kWave + lane) * 8;
        if (c < cols) {
          float wv[8], xv[8], gv[8];
          Elem<T>::load8(w + c, wv);
          Elem<T>::unpack(xr[k][i], xv);
          Elem<T>::unpack(gr[k][i], gv);
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float n = xv[j] * r;
            dn[i][j] = Elem<T>::rnd(gv[j] * wv[j]);
            acc[i][j] = fmaf(gv[j], Elem<T>::rnd(n), acc[i][j]);
            dot = fmaf(dn[i][j], n, dot);
          }
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) dn[i][j] = 0.f;
        }
      }
      dot = wave_sum(dot) * inv_cols;
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int c = (i * kWave + lane) * 8;
        if (c < cols) {
          float xv[8], o[8];
          Elem<T>::unpack(xr[k][i], xv);
#pragma unroll
          for (int j = 0; j < 8; ++j) o[j] = r * (dn[i][j] - xv[j] * r * dot);
          if constexpr (RES) {
            float rv[8];
            Elem<T>::unpack(rr[k][i], rv);
#pragma unroll
            for (int j = 0; j < 8; ++j) o[j] += rv[j];
          }
          Elem<T>::store8(dx + base + c, o);
        }
      }
    }
  }

  // Fixed-order combination of the 4 per-wave partials.
  for (int wv = 0; wv < kRowsPerBlock; ++wv) {
    if (wave == wv) {
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int c = (i * kWave + lane) * 8;
        if (c < cols) {
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            if (wv == 0) lds_acc[c + j] = acc[i][j];
            else lds_acc[c + j] += acc[i][j];
          }
        }
      }
    }
    __syncthreads();
  }
  float* dst = part + static_cast<int64_t>(blockIdx.x) * cols;
  for (int c = threadIdx.x; c < cols; c += blockDim.x) dst[c] = lds_acc[c];
}

// dw[c] = sum_p part[p, c]; block = 64 columns x 16 waves, fixed order.  Each
// wave keeps 8 independent partial-row loads in flight.
template <typename T>
__global__ __launch_bounds__(1024) void k_reduce_cols(const float* __restrict__ part,
                                                      int nparts, int cols,
                                                      T* __restrict__ out) {
  __shared__ float red[16][65];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c = blockIdx.x * 64 + lane;
  float s = 0.f;
  if (c < cols) {
    int p = wave;
    for (; p + 16 * 7 < nparts; p += 16 * 8) {
      float v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = part[static_cast<int64_t>(p + 16 * k) * cols + c];
#pragma unroll
      for (int k = 0; k < 8; ++k) s += v[k];
    }
    for (; p < nparts; p += 16) s += part[static_cast<int64_t>(p) * cols + c];
  }
  red[wave][lane] = s;
  __syncthreads();
  if (wave == 0 && c < cols) {
    float t = 0.f;
    for (int k = 0; k < 16; ++k) t += red[k][lane];
    Elem<T>::st1(out + c, t);
  }
}

// Backward grid cap: fewer blocks mean fewer fp32 dw partial rows for
// k_reduce_cols; 512 blocks measured best at T=16384, H=2048 (4.05 TB/s for
// both kernels together vs 3.43 at 1024 and 3.74 at 256).
#ifndef FH_NORM_BWD_BLOCKS
#define FH_NORM_BWD_BLOCKS 512
#endif
constexpr int kMaxBwdBlocks = FH_NORM_BWD_BLOCKS;

int bwd_blocks(int64_t rows) {
  const int64_t need = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
  return static_cast<int>(need < kMaxBwdBlocks ? need : kMaxBwdBlocks);
}

template <typename T, int NV>
void launch_fwd(const void* x, const void* a, const void* w, void* h, void* y, float* rstd,
                int64_t rows, int cols, float eps, hipStream_t s) {
  const int64_t per_block = static_cast<int64_t>(kRowsPerBlock) * FwdRows<NV>::R;
  const dim3 grid(static_cast<unsigned>((rows + per_block - 1) / per_block));
  if (a != nullptr) {
    hipLaunchKernelGGL((k_rmsnorm_fwd<T, NV, true>), grid, dim3(256), 0, s,
                       static_cast<const T*>(x), static_cast<const T*>(a),
                       static_cast<const T*>(w), static_cast<T*>(h), static_cast<T*>(y), rstd,
                       rows, cols, eps);
  } else {
    hipLaunchKernelGGL((k_rmsnorm_fwd<T, NV, false>), grid, dim3(256), 0, s,
                       static_cast<const T*>(x), nullptr, static_cast<const T*>(w), nullptr,
                       static_cast<T*>(y), rstd, rows, cols, eps);
  }
}

template <typename T, int NV, bool RES, bool HR>
void launch_bwd_k(const void* dy, const void* x, const void* w, const float* rstd,
                  const void* dres, void* dx, float* part, int64_t rows, int cols, float eps,
                  int blocks, hipStream_t s) {
  hipLaunchKernelGGL((k_rmsnorm_bwd<T, NV, RES, HR>), dim3(blocks), dim3(256),
                     static_cast<size_t>(cols) * sizeof(float), s, static_cast<const T*>(dy),
                     static_cast<const T*>(x), static_cast<const T*>(w), rstd,
                     static_cast<const T*>(dres), static_cast<T*>(dx), part, rows, cols, eps);
}

template <typename T, int NV>
void launch_bwd(const void* dy, const void* x, const void* w, const float* rstd,
                const void* dres, void* dx, void* dw, float* part, int64_t rows, int cols,
                float eps, hipStream_t s) {
  const int blocks = bwd_blocks(rows);
  const bool res = dres != nullptr, hr = rstd != nullptr;
  if (res && hr) launch_bwd_k<T, NV, true, true>(dy, x, w, rstd, dres, dx, part, rows, cols, eps, blocks, s);
  else if (res) launch_bwd_k<T, NV, true, false>(dy, x, w, rstd, dres, dx, part, rows, cols, eps, blocks, s);
  else if (hr) launch_bwd_k<T, NV, false, true>(dy, x, w, rstd, dres, dx, part, rows, cols, eps, blocks, s);
  else launch_bwd_k<T, NV, false, false>(dy, x, w, rstd, dres, dx, part, rows, cols, eps, blocks, s);
  hipLaunchKernelGGL((k_reduce_cols<T>), dim3((cols + 63) / 64), dim3(1024), 0, s, part, blocks,
                     cols, static_cast<T*>(dw));
}

// Chunks of 8 per lane: cols <= 512*NV.
template <typename F>
int dispatch_nv(int cols, F&& f) {
  if (cols <= 512) return f(std::integral_constant<int, 1>{});
  if (cols <= 1024) return f(std::integral_constant<int, 2>{});
  if (cols <= 2048) return f(std::integral_constant<int, 4>{});
  if (cols <= 4096) return f(std::integral_constant<int, 8>{});
  return f(std::integral_constant<int, 16>{});
}

int validate_rows(fh_dtype dt, int64_t rows, int64_t cols) {
  FH_REQUIRE(dt == FH_BF16 || dt == FH_F32, "rmsnorm: dtype must be FH_BF16 or FH_F32");
  FH_REQUIRE(rows >= 0, "rmsnorm: rows must be >= 0");
  FH_REQUIRE(cols > 0 && cols % 8 == 0 && cols <= 8192,
             "rmsnorm: cols must be a positive multiple of 8 and <= 8192");
  return FH_OK;
}

}  // namespace
}  // namespace fh

using namespace fh;

extern "C" int fh_rmsnorm_fwd(fh_dtype dt, const void* x, const void* w, void* y, float* rstd,
                              int64_t rows, int64_t cols, float eps, hipStream_t stream) {
  if (int e = validate_rows(dt, rows, cols)) return e;
  if (rows == 0) return FH_OK;
  FH_REQUIRE(x && w && y, "rmsnorm_fwd: null pointer");
  FH_REQUIRE(aligned16(x) && aligned16(w) && aligned16(y), "rmsnorm_fwd: pointers must be 16-byte aligned");
  const int c = static_cast<int>(cols);
  dispatch_nv(c, [&](auto nv) {
    if (dt == FH_BF16) launch_fwd<uint16_t, nv()>(x, nullptr, w, nullptr, y, rstd, rows, c, eps, stream);
    else launch_fwd<float, nv()>(x, nullptr, w, nullptr, y, rstd, rows, c, eps, stream);
    return 0;
  });
  return check_launch("fh_rmsnorm_fwd");
}

extern "C" int fh_add_rmsnorm_fwd(fh_dtype dt, const void* x, const void* a, const void* w,
                                  void* h, void* y, float* rstd, int64_t rows, int64_t cols,
                                  float eps, hipStream_t stream) {
  if (int e = validate_rows(dt, rows, cols)) return e;
  if (rows == 0) return FH_OK;
  FH_REQUIRE(x && a && w && h && y, "add_rmsnorm_fwd: null pointer");
  FH_REQUIRE(aligned16(x) && aligned16(a) && aligned16(w) && aligned16(h) && aligned16(y),
             "add_rmsnorm_fwd: pointers must be 16-byte aligned");
  FH_REQUIRE(h != x && h != a, "add_rmsnorm_fwd: h must not alias x or a");
  const int c = static_cast<int>(cols);
  dispatch_nv(c, [&](auto nv) {
    if (dt == FH_BF16) launch_fwd<uint16_t, nv()>(x, a, w, h, y, rstd, rows, c, eps, stream);
    else launch_fwd<float, nv()>(x, a, w, h, y, rstd, rows, c, eps, stream);
    return 0;
  });
  return check_launch("fh_add_rmsnorm_fwd");
}

extern "C" size_t fh_rmsnorm_bwd_workspace_size(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return 0;
  return static_cast<size_t>(bwd_blocks(rows)) * static_cast<size_t>(cols) * sizeof(float);
}

extern "C" int fh_rmsnorm_bwd(fh_dtype dt, const void* dy, const void* x, const void* w,
                              const float* rstd, const void* dres, void* dx, void* dw,
                              void* workspace, int64_t rows, int64_t cols, float eps,
                              hipStream_t stream) {
  if (int e = validate_rows(dt, rows, cols)) return e;
  FH_REQUIRE(w && dw, "rmsnorm_bwd: null pointer");
  const int c = static_cast<int>(cols);
  if (rows == 0) {
    // Empty batch: the weight gradient is an all-zero row (a reduction over
    // zero partials; a kernel rather than hipMemsetAsync so the call stays
    // safe inside a captured graph).
    if (dt == FH_BF16)
      hipLaunchKernelGGL((k_reduce_cols<uint16_t>), dim3((c + 63) / 64), dim3(1024), 0, stream,
                         nullptr, 0, c, static_cast<uint16_t*>(dw));
    else
      hipLaunchKernelGGL((k_reduce_cols<float>), dim3((c + 63) / 64), dim3(1024), 0, stream,
                         nullptr, 0, c, static_cast<float*>(dw));
    return check_launch("fh_rmsnorm_bwd");
  }
  FH_REQUIRE(dy && x && dx && workspace, "rmsnorm_bwd: null pointer");
  FH_REQUIRE(aligned16(dy) && aligned16(x) && aligned16(w) && aligned16(dx) &&
                 (dres == nullptr || aligned16(dres)),
             "rmsnorm_bwd: pointers must be 16-byte aligned");
  float* part = static_cast<float*>(workspace);
  dispatch_nv(c, [&](auto nv) {
    if (dt == FH_BF16) launch_bwd<uint16_t, nv()>(dy, x, w, rstd, dres, dx, dw, part, rows, c, eps, stream);
    else launch_bwd<float, nv()>(dy, x, w, rstd, dres, dx, dw, part, rows, c, eps, stream);
    return 0;
  });
  return check_launch("fh_rmsnorm_bwd");
}
