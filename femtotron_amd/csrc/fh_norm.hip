// RMSNorm forward / residual-add + RMSNorm forward / RMSNorm backward.
//
// Reference arithmetic: LlamaRMSNorm.forward, transformers 5.15.0
// models/llama/modeling_llama.py:62-67, and the residual adds at :317/:323.
//
// Layout: lane l of a wave owns the 8-element chunks starting at columns
// (i*64 + l)*8 of its share of a row, so each load instruction of a wave
// covers one contiguous 1 KiB (bf16) span; rows stay in registers, packed as
// loaded, between the reduction and the normalisation, so every input is read
// from HBM exactly once.  The weight row is loaded once per wave, together
// with the first data, so its latency is never on a row's critical path.
#include "fh_common.hpp"

#include <mutex>

namespace fh {
namespace {

constexpr int kWavesPerBlock = 4;  // 256 threads

// Forward: one wave per R consecutive rows (all loads of the R rows issued
// before the first reduction).
#ifndef FH_NORM_FWD_ROWS
#define FH_NORM_FWD_ROWS 1
#endif
template <int NV>
struct FwdRows {
  static constexpr int R = NV <= 4 ? FH_NORM_FWD_ROWS : 1;
};

template <typename T, int NV, bool ADD, int R>
__global__ __launch_bounds__(256) void k_rmsnorm_fwd(
    const T* __restrict__ x, const T* __restrict__ a, const T* __restrict__ w,
    T* __restrict__ h, T* __restrict__ y, float* __restrict__ rstd,
    int64_t rows, int cols, float eps) {
  using Raw = typename Elem<T>::Raw;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + (threadIdx.x >> 6)) * R;
  if (row0 >= rows) return;  // uniform per wave

  Raw xr[R][NV], wr[NV];
  [[maybe_unused]] Raw ar[R][NV];
#pragma unroll
  for (int k = 0; k < R; ++k) {
    const int64_t base = (row0 + k) * cols;
    const bool ok = row0 + k < rows;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = (i * kWave + lane) * 8;
      if (ok && c < cols) {
        xr[k][i] = Elem<T>::ldraw(x + base + c);
        if constexpr (ADD) ar[k][i] = Elem<T>::ldraw(a + base + c);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = (i * kWave + lane) * 8;
    if (c < cols) wr[i] = Elem<T>::ldraw(w + c);
  }
#pragma unroll
  for (int k = 0; k < R; ++k) {
    if (row0 + k >= rows) break;  // uniform per wave
    const int64_t base = (row0 + k) * cols;
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = (i * kWave + lane) * 8;
      if (c < cols) {
        float v[8];
        Elem<T>::unpack(xr[k][i], v);
        if constexpr (ADD) {  // h = to_dtype(x + a), kept packed for the normalisation
          float b[8];
          Elem<T>::unpack(ar[k][i], b);
#pragma unroll
          for (int j = 0; j < 8; ++j) v[j] = Elem<T>::rnd(v[j] + b[j]);
          xr[k][i] = Elem<T>::pack(v);
          Elem<T>::straw(h + base + c, xr[k][i]);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) ss = fmaf(v[j], v[j], ss);
      }
    }
    ss = wave_sum(ss);
    const float r = rsqrtf(ss / static_cast<float>(cols) + eps);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = (i * kWave + lane) * 8;
      if (c < cols) {
        float v[8], wv[8], o[8];
        Elem<T>::unpack(xr[k][i], v);
        Elem<T>::unpack(wr[i], wv);
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = Elem<T>::rnd(wv[j] * Elem<T>::rnd(v[j] * r));
        Elem<T>::store8(y + base + c, o);
      }
    }
    if (rstd != nullptr && lane == 0) rstd[row0 + k] = r;
  }
}

// Backward.  WPR waves share a row (WPR = 2 above 2048 columns), each holding
// NVW chunks of 8 per lane, so every width keeps the register footprint of a
// 2048-column row.  A block's 4 waves take 4/WPR rows per step; the step loop
// is uniform across the block (its barriers combine the WPR per-wave partial
// sums of a row in a fixed order, through a parity-double-buffered LDS slot).
// Per row:
//   r   = rstd (given) or rsqrt(mean(x^2) + eps)
//   dn  = to_dtype(dy * w)          (the gradient at the bf16 normalised value)
//   dot = mean(dn * x * r)
//   dx  = r * (dn - x * r * dot) [+ dres]
//   dw += dy * to_dtype(x * r)      (per-wave registers)
// The weight-gradient partials of the block's waves are summed in a fixed
// order through LDS into one fp32 row per block (deterministic), which
// k_reduce_parts / k_reduce_stage fold into dw.
// Next-row prefetch (PF): measured 50.6 -> 43.5 us without the residual
// gradient at T=16384, H=2048; with it (3 input rows) the extra registers cost
// a wave of occupancy and it gained nothing (60.8 vs 62.3 us), so it is on only
// for the 2-input form.
template <typename T, int NVW, int WPR, int NWB, bool RES, bool HAVE_RSTD, bool PF = !RES>
__global__ __launch_bounds__(64 * NWB) void k_rmsnorm_bwd(
    const T* __restrict__ dy, const T* __restrict__ x, const T* __restrict__ w,
    const float* __restrict__ rstd, const T* __restrict__ dres,
    T* __restrict__ dx, float* __restrict__ part, int64_t rows, int cols,
    float eps) {
  using Raw = typename Elem<T>::Raw;
  constexpr int RPB = NWB / WPR;  // rows per block step (NWB waves per block)
  extern __shared__ float lds_acc[];          // cols floats
  __shared__ float red[2][2][NWB];  // [step parity][ss | dot][wave]
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;
  const int rsub = wave / WPR, slice = wave % WPR;
  auto col = [&](int i) { return ((slice * NVW + i) * kWave + lane) * 8; };

  Raw wr[NVW];
#pragma unroll
  for (int i = 0; i < NVW; ++i)
    if (col(i) < cols) wr[i] = Elem<T>::ldraw(w + col(i));
  float acc[NVW][8];
#pragma unroll
  for (int i = 0; i < NVW; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = 0.f;

  const float inv_cols = 1.f / static_cast<float>(cols);
  const int64_t stride = static_cast<int64_t>(gridDim.x) * RPB;
  // Loads of one row; with PF the next step's row is loaded while this one is
  // processed (two rows of this wave in flight).
  Raw xn[NVW], gn[NVW];
  [[maybe_unused]] Raw rn[NVW];
  auto load_row = [&](int64_t row) {
    if (row >= rows) return;
    const int64_t base = row * cols;
#pragma unroll
    for (int i = 0; i < NVW; ++i) {
      const int c = col(i);
      if (c < cols) {
        xn[i] = Elem<T>::ldraw(x + base + c);
        gn[i] = Elem<T>::ldraw(dy + base + c);
        if constexpr (RES) rn[i] = Elem<T>::ldraw(dres + base + c);
      }
    }
  };
  int par = 0;
  if constexpr (PF) load_row(static_cast<int64_t>(blockIdx.x) * RPB + rsub);
  for (int64_t step0 = static_cast<int64_t>(blockIdx.x) * RPB; step0 < rows;
       step0 += stride, par ^= 1) {
    const int64_t row = step0 + rsub;
    const bool valid = row < rows;  // uniform per wave
    const int64_t base = row * cols;
    if constexpr (!PF) load_row(row);
    Raw xr[NVW], gr[NVW];
    [[maybe_unused]] Raw rr[NVW];
#pragma unroll
    for (int i = 0; i < NVW; ++i) {
      xr[i] = xn[i];
      gr[i] = gn[i];
      if constexpr (RES) rr[i] = rn[i];
    }
    if constexpr (PF) load_row(row + stride);
    float r;
    if constexpr (HAVE_RSTD) {
      r = valid ? rstd[row] : 0.f;
    } else {
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < NVW; ++i) {
        if (valid && col(i) < cols) {
          float xv[8];
          Elem<T>::unpack(xr[i], xv);
#pragma unroll
          for (int j = 0; j < 8; ++j) ss = fmaf(xv[j], xv[j], ss);
        }
      }
      ss = wave_sum(ss);
      if constexpr (WPR > 1) {
        if (lane == 0) red[par][0][wave] = ss;
        __syncthreads();
        ss = 0.f;
#pragma unroll
        for (int s = 0; s < WPR; ++s) ss += red[par][0][rsub * WPR + s];
      }
      r = rsqrtf(ss * inv_cols + eps);
    }
    float dot = 0.f;
#pragma unroll
    for (int i = 0; i < NVW; ++i) {
      if (valid && col(i) < cols) {
        float wv[8], xv[8], gv[8];
        Elem<T>::unpack(wr[i], wv);
        Elem<T>::unpack(xr[i], xv);
        Elem<T>::unpack(gr[i], gv);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float n = xv[j] * r;
          dot = fmaf(Elem<T>::rnd(gv[j] * wv[j]), n, dot);
          acc[i][j] = fmaf(gv[j], Elem<T>::rnd(n), acc[i][j]);
        }
      }
    }
    dot = wave_sum(dot);
    if constexpr (WPR > 1) {
      if (lane == 0) red[par][1][wave] = dot;
      __syncthreads();
      dot = 0.f;
#pragma unroll
      for (int s = 0; s < WPR; ++s) dot += red[par][1][rsub * WPR + s];
    }
    dot *= inv_cols;
#pragma unroll
    for (int i = 0; i < NVW; ++i) {
      const int c = col(i);
      if (valid && c < cols) {
        float wv[8], xv[8], gv[8], o[8];
        Elem<T>::unpack(wr[i], wv);
        Elem<T>::unpack(xr[i], xv);
        Elem<T>::unpack(gr[i], gv);
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = r * (Elem<T>::rnd(gv[j] * wv[j]) - xv[j] * r * dot);
        if constexpr (RES) {
          float rv[8];
          Elem<T>::unpack(rr[i], rv);
#pragma unroll
          for (int j = 0; j < 8; ++j) o[j] += rv[j];
        }
        Elem<T>::store8(dx + base + c, o);
      }
    }
  }

  // Fixed-order combination of the per-wave partials (waves with the same
  // slice cover the same columns; row groups rsub = 0, 1, ... in order).
  for (int s = 0; s < RPB; ++s) {
    if (rsub == s) {
#pragma unroll
      for (int i = 0; i < NVW; ++i) {
        const int c = col(i);
        if (c < cols) {
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            if (s == 0) lds_acc[c + j] = acc[i][j];
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

// dw[c] = sum_p part[p, c], deterministic, in two stages.  Stage 1: block
// (cx, g) sums partial rows p = g, g + G, g + 2G, ... (each of its 4 waves
// takes every 4th of them, all loads in flight at once) for 64 columns and
// combines its waves in a fixed order into stage[g][c].  Stage 2 sums the G
// stage rows of a column in order.  The partial rows are few (<= 512) and
// wide, so one stage would leave the reduction latency-bound on a handful of
// CUs.
constexpr int kReduceGroups = 16;

__global__ __launch_bounds__(256) void k_reduce_parts(const float* __restrict__ part, int nparts,
                                                      int cols, float* __restrict__ stage) {
  __shared__ float red[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = blockIdx.x * 64 + lane, g = blockIdx.y;
  float s = 0.f;
  if (c < cols) {
    constexpr int U = 8;  // loads in flight per lane
    int p = g + kReduceGroups * wave;
    for (; p + kReduceGroups * 4 * (U - 1) < nparts; p += kReduceGroups * 4 * U) {
      float v[U];
#pragma unroll
      for (int k = 0; k < U; ++k) v[k] = part[static_cast<int64_t>(p + kReduceGroups * 4 * k) * cols + c];
#pragma unroll
      for (int k = 0; k < U; ++k) s += v[k];
    }
    for (; p < nparts; p += kReduceGroups * 4) s += part[static_cast<int64_t>(p) * cols + c];
  }
  red[wave][lane] = s;
  __syncthreads();
  if (wave == 0 && c < cols)
    stage[static_cast<int64_t>(g) * cols + c] = ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane];
}

template <typename T>
__global__ __launch_bounds__(256) void k_fill_zero(T* __restrict__ out, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) Elem<T>::st1(out + i, 0.f);
}

template <typename T>
__global__ __launch_bounds__(256) void k_reduce_stage(const float* __restrict__ stage, int cols,
                                                      T* __restrict__ out) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= cols) return;
  float t = 0.f;
#pragma unroll
  for (int g = 0; g < kReduceGroups; ++g) t += stage[static_cast<int64_t>(g) * cols + c];
  Elem<T>::st1(out + c, t);
}

// Backward grid cap: fewer blocks mean fewer fp32 dw partial rows to reduce;
// 512 measured best at T=16384, H=2048 (256 and 1024 both slower).
#ifndef FH_NORM_BWD_BLOCKS
#define FH_NORM_BWD_BLOCKS 512
#endif
constexpr int kMaxBwdBlocks = FH_NORM_BWD_BLOCKS;

template <typename T, int NV>
void launch_fwd(const void* x, const void* a, const void* w, void* h, void* y, float* rstd,
                int64_t rows, int cols, float eps, hipStream_t s) {
  constexpr int R = FwdRows<NV>::R;
  const int64_t per_block = static_cast<int64_t>(kWavesPerBlock) * R;
  const dim3 grid(static_cast<unsigned>((rows + per_block - 1) / per_block));
  if (a != nullptr) {
    hipLaunchKernelGGL((k_rmsnorm_fwd<T, NV, true, R>), grid, dim3(256), 0, s,
                       static_cast<const T*>(x), static_cast<const T*>(a),
                       static_cast<const T*>(w), static_cast<T*>(h), static_cast<T*>(y), rstd,
                       rows, cols, eps);
  } else {
    hipLaunchKernelGGL((k_rmsnorm_fwd<T, NV, false, R>), grid, dim3(256), 0, s,
                       static_cast<const T*>(x), nullptr, static_cast<const T*>(w), nullptr,
                       static_cast<T*>(y), rstd, rows, cols, eps);
  }
}

// Backward row split: WPR waves per row, NVW chunks of 8 per lane, NWB waves
// per block (RPB = NWB / WPR rows per block step).  Rows of 1025-2048 columns
// with the residual gradient (the layer's two norms) take two waves each in
// blocks of 8: twice the waves in flight at the same partial-row count, 60 ->
// 56 us at T = 16384, H = 2048 (one wave per row in blocks of 8 or 16 needs
// more than the 128 registers of four waves per SIMD).
template <int NV, bool RES>
struct BwdSplit {
  static constexpr int WPR = NV > 4 || (NV == 4 && RES) ? 2 : 1;
  static constexpr int NVW = NV / WPR;
  static constexpr int NWB = NV == 4 && RES ? 8 : 4;
  static constexpr int RPB = NWB / WPR;
};

// Blocks of the backward: one per RPB rows, at most kMaxBwdBlocks (each
// writes one fp32 partial row of dw).
int bwd_blocks(int64_t rows, int rpb) {
  const int64_t need = (rows + rpb - 1) / rpb;
  return static_cast<int>(need < kMaxBwdBlocks ? need : kMaxBwdBlocks);
}

template <typename T, int NV, bool RES, bool HR>
void launch_bwd_k(const void* dy, const void* x, const void* w, const float* rstd,
                  const void* dres, void* dx, float* part, int64_t rows, int cols, float eps,
                  int blocks, hipStream_t s) {
  using SP = BwdSplit<NV, RES>;
  hipLaunchKernelGGL((k_rmsnorm_bwd<T, SP::NVW, SP::WPR, SP::NWB, RES, HR>), dim3(blocks), dim3(64 * SP::NWB),
                     static_cast<size_t>(cols) * sizeof(float), s, static_cast<const T*>(dy),
                     static_cast<const T*>(x), static_cast<const T*>(w), rstd,
                     static_cast<const T*>(dres), static_cast<T*>(dx), part, rows, cols, eps);
}

template <typename T, int NV>
void launch_bwd(const void* dy, const void* x, const void* w, const float* rstd,
                const void* dres, void* dx, void* dw, float* part, int64_t rows, int cols,
                float eps, hipStream_t s) {
  const bool res = dres != nullptr, hr = rstd != nullptr;
  const int blocks = bwd_blocks(rows, res ? BwdSplit<NV, true>::RPB : BwdSplit<NV, false>::RPB);
  if (res && hr) launch_bwd_k<T, NV, true, true>(dy, x, w, rstd, dres, dx, part, rows, cols, eps, blocks, s);
  else if (res) launch_bwd_k<T, NV, true, false>(dy, x, w, rstd, dres, dx, part, rows, cols, eps, blocks, s);
  else if (hr) launch_bwd_k<T, NV, false, true>(dy, x, w, rstd, dres, dx, part, rows, cols, eps, blocks, s);
  else launch_bwd_k<T, NV, false, false>(dy, x, w, rstd, dres, dx, part, rows, cols, eps, blocks, s);
  float* stage = part + static_cast<int64_t>(blocks) * cols;
  hipLaunchKernelGGL(k_reduce_parts, dim3((cols + 63) / 64, kReduceGroups), dim3(256), 0, s, part,
                     blocks, cols, stage);
  hipLaunchKernelGGL((k_reduce_stage<T>), dim3((cols + 255) / 256), dim3(256), 0, s, stage, cols,
                     static_cast<T*>(dw));
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
  // one fp32 partial row per backward block (4 rows per block, 2 above 2048
  // columns), then the reduction's stage rows
  const int64_t nrows = bwd_blocks(rows, cols > 2048 ? 2 : 4) + kReduceGroups;
  return static_cast<size_t>(nrows) * static_cast<size_t>(cols) * sizeof(float);
}

namespace fh {
namespace {

// Scratch of the allocation-free backward: the fp32 partial rows of the
// largest valid call (kMaxBwdBlocks partial rows + kReduceGroups stage rows of
// at most 8192 columns), 17.3 MB per device, held until the process ends.
constexpr size_t kNoAllocScratchFloats = static_cast<size_t>(kMaxBwdBlocks + kReduceGroups) * 8192;
__device__ __align__(256) float scratch[kNoAllocScratchFloats];

// Device address of `scratch` on the current device, looked up once per
// device (each device holds its own copy of the array at its own address;
// the host-side symbol is only a stand-in and must never reach a kernel).
float* scratch_on_current_device(int* status) {
  constexpr int kMaxDevices = 64;
  static std::once_flag once[kMaxDevices];
  static float* addr[kMaxDevices] = {};
  static hipError_t err[kMaxDevices] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    *status = fail(FH_ERR_LAUNCH, "rmsnorm_bwd_noalloc: no current HIP device");
    return nullptr;
  }
  std::call_once(once[dev], [dev]() {
    void* p = nullptr;
    err[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    addr[dev] = static_cast<float*>(p);
  });
  if (err[dev] != hipSuccess || addr[dev] == nullptr) {
    *status = fail(FH_ERR_LAUNCH, std::string("rmsnorm_bwd_noalloc: hipGetSymbolAddress failed: ") +
                                      hipGetErrorString(err[dev]));
    return nullptr;
  }
  *status = FH_OK;
  return addr[dev];
}

}  // namespace
}  // namespace fh

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
      hipLaunchKernelGGL((k_fill_zero<uint16_t>), dim3((c + 255) / 256), dim3(256), 0, stream,
                         static_cast<uint16_t*>(dw), c);
    else
      hipLaunchKernelGGL((k_fill_zero<float>), dim3((c + 255) / 256), dim3(256), 0, stream,
                         static_cast<float*>(dw), c);
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

extern "C" size_t fh_rmsnorm_bwd_noalloc_max_workspace(void) {
  return kNoAllocScratchFloats * sizeof(float);
}

extern "C" int fh_rmsnorm_bwd_noalloc(fh_dtype dt, const void* dy, const void* x, const void* w,
                                      const float* rstd, const void* dres, void* dx, void* dw,
                                      int64_t rows, int64_t cols, float eps, hipStream_t stream) {
  if (int e = validate_rows(dt, rows, cols)) return e;
  FH_REQUIRE(fh_rmsnorm_bwd_workspace_size(rows, cols) <= kNoAllocScratchFloats * sizeof(float),
             "rmsnorm_bwd_noalloc: the call needs more scratch than the library holds");
  if (rows == 0)  // no scratch needed: dw = 0
    return fh_rmsnorm_bwd(dt, dy, x, w, rstd, dres, dx, dw, nullptr, rows, cols, eps, stream);
  int status = FH_OK;
  float* ws = scratch_on_current_device(&status);
  if (ws == nullptr) return status;
  return fh_rmsnorm_bwd(dt, dy, x, w, rstd, dres, dx, dw, ws, rows, cols, eps, stream);
}
