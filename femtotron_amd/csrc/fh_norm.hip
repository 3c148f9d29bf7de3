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

// Forward: each wave takes rows row, row + stride, ... (stride = 4 x grid).
// With PIPE the next row's loads are issued before this row is reduced and
// stored, so a wave keeps two rows in flight; without it the grid covers every
// row once (one row per wave).  The pipelined form is used for add+RMSNorm
// (two input rows): 45.2 -> 43.1 us at T = 16384, H = 2048 and 50.5 -> 48.8 us
// at T = 8192, H = 4096; the one-input form measured no gain from it.
template <typename T, int NV, bool ADD, bool PIPE>
__global__ __launch_bounds__(256) void k_rmsnorm_fwd(
    const T* __restrict__ x, const T* __restrict__ a, const T* __restrict__ w,
    T* __restrict__ h, T* __restrict__ y, float* __restrict__ rstd,
    int64_t rows, int cols, float eps) {
  using Raw = typename Elem<T>::Raw;
  const int lane = threadIdx.x & (kWave - 1);
  int64_t row = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + (threadIdx.x >> 6);
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kWavesPerBlock;
  if (row >= rows) return;  // uniform per wave

  Raw xn[NV], wr[NV];
  [[maybe_unused]] Raw an[NV];
  auto load_row = [&](int64_t rr) {
    const int64_t base = rr * cols;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = (i * kWave + lane) * 8;
      if (c < cols) {
        xn[i] = Elem<T>::ldraw(x + base + c);
        if constexpr (ADD) an[i] = Elem<T>::ldraw(a + base + c);
      }
    }
  };
  load_row(row);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = (i * kWave + lane) * 8;
    if (c < cols) wr[i] = Elem<T>::ldraw(w + c);
  }
  // Normalises row rr from its loaded chunks (xr, and ar with ADD).
  auto norm_row = [&](int64_t rr, Raw* xr, [[maybe_unused]] Raw* ar) {
    const int64_t base = rr * cols;
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = (i * kWave + lane) * 8;
      if (c < cols) {
        float v[8];
        Elem<T>::unpack(xr[i], v);
        if constexpr (ADD) {  // h = to_dtype(x + a), kept packed for the normalisation
          float b[8];
          Elem<T>::unpack(ar[i], b);
#pragma unroll
          for (int j = 0; j < 8; ++j) v[j] = Elem<T>::rnd(v[j] + b[j]);
          xr[i] = Elem<T>::pack(v);
          Elem<T>::straw(h + base + c, xr[i]);
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
        Elem<T>::unpack(xr[i], v);
        Elem<T>::unpack(wr[i], wv);
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = Elem<T>::rnd(wv[j] * Elem<T>::rnd(v[j] * r));
        Elem<T>::store8(y + base + c, o);
      }
    }
    if (rstd != nullptr && lane == 0) rstd[rr] = r;
  };
  if constexpr (!PIPE) {
    norm_row(row, xn, an);
  } else {
    for (; row < rows; row += stride) {  // uniform per wave
      Raw xr[NV];
      [[maybe_unused]] Raw ar[NV];
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        xr[i] = xn[i];
        if constexpr (ADD) ar[i] = an[i];
      }
      if (row + stride < rows) load_row(row + stride);
      norm_row(row, xr, ar);
    }
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
// k_reduce_parts folds into dw.
// Next-row prefetch (PF): measured 50.6 -> 43.5 us without the residual
// gradient at T=16384, H=2048; with it (3 input rows) at that width the extra
// registers cost a wave of occupancy and it gained nothing (60.8 vs 62.3 us);
// BwdSplit chooses it per width.
template <typename T, int NVW, int WPR, int NWB, bool RES, bool HAVE_RSTD, bool PF>
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

// dw[c] = sum_p part[p, c], deterministic, in one launch.  A block owns 16
// columns: its 256 threads are 64 row groups x 4 column quads; thread (g, q)
// sums the float4 of rows p = g, g + 64, g + 128, ... in order (eight loads in
// flight), and the 64 group sums of a column are added in group order.  One
// launch instead of a partial pass plus a stage pass measured 1-2 us faster
// per backward call (one launch gap fewer).
template <typename T>
__global__ __launch_bounds__(256) void k_reduce_parts(const float* __restrict__ part, int nparts,
                                                      int cols, T* __restrict__ out) {
  constexpr int G = 64, U = 8;
  __shared__ float red[G][17];
  const int q = threadIdx.x & 3, g = threadIdx.x >> 2;
  const int c = blockIdx.x * 16 + q * 4;  // cols % 8 == 0: a quad is wholly in or out
  float4 s = {0.f, 0.f, 0.f, 0.f};
  if (c < cols) {
    auto at = [&](int p) {
      return *reinterpret_cast<const float4*>(part + static_cast<int64_t>(p) * cols + c);
    };
    int p = g;
    for (; p + G * (U - 1) < nparts; p += G * U) {
      float4 v[U];
#pragma unroll
      for (int k = 0; k < U; ++k) v[k] = at(p + G * k);
#pragma unroll
      for (int k = 0; k < U; ++k) {
        s.x += v[k].x; s.y += v[k].y; s.z += v[k].z; s.w += v[k].w;
      }
    }
    for (; p < nparts; p += G) {
      const float4 v = at(p);
      s.x += v.x; s.y += v.y; s.z += v.z; s.w += v.w;
    }
  }
  red[g][q * 4 + 0] = s.x;
  red[g][q * 4 + 1] = s.y;
  red[g][q * 4 + 2] = s.z;
  red[g][q * 4 + 3] = s.w;
  __syncthreads();
  const int cc = blockIdx.x * 16 + static_cast<int>(threadIdx.x);
  if (threadIdx.x < 16 && cc < cols) {
    float t = 0.f;
    for (int k = 0; k < G; ++k) t += red[k][threadIdx.x];
    Elem<T>::st1(out + cc, t);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void k_fill_zero(T* __restrict__ out, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) Elem<T>::st1(out + i, 0.f);
}

// Backward grid cap: fewer blocks mean fewer fp32 dw partial rows to reduce;
// 512 measured best at T=16384, H=2048 (256 and 1024 both slower).
#ifndef FH_NORM_BWD_BLOCKS
#define FH_NORM_BWD_BLOCKS 512
#endif
constexpr int kMaxBwdBlocks = FH_NORM_BWD_BLOCKS;

// Grid cap of the pipelined add+RMSNorm forward (768 measured best of 512,
// 768, 1024 and 2048 at T = 16384, H = 2048).
constexpr int64_t kFwdPipeBlocks = 768;
// Grid cap of the pipelined one-input forward (2049-4096 bf16 columns).
constexpr int64_t kFwdPipeBlocks1 = 512;

template <typename T, int NV>
void launch_fwd(const void* x, const void* a, const void* w, void* h, void* y, float* rstd,
                int64_t rows, int cols, float eps, hipStream_t s) {
  const int64_t need = (rows + kWavesPerBlock - 1) / kWavesPerBlock;
  if (a != nullptr) {
    // add+RMSNorm: pipelined over a capped grid where the two rows of x and a
    // in flight fit the registers (bf16 up to 4096 columns, fp32 up to 2048)
    constexpr bool kPipe = NV * sizeof(typename Elem<T>::Raw) <= 128;
    const dim3 grid(static_cast<unsigned>(kPipe && need > kFwdPipeBlocks ? kFwdPipeBlocks : need));
    hipLaunchKernelGGL((k_rmsnorm_fwd<T, NV, true, kPipe>), grid, dim3(256), 0, s,
                       static_cast<const T*>(x), static_cast<const T*>(a),
                       static_cast<const T*>(w), static_cast<T*>(h), static_cast<T*>(y), rstd,
                       rows, cols, eps);
  } else if (NV == 8 && sizeof(typename Elem<T>::Raw) == 16 && need > kFwdPipeBlocks1) {
    // one input, 2049-4096 bf16 columns: pipelined over a capped grid (kernel
    // time 15.3 -> 14.1 us at T = 4096, 26.1 -> 23.7 us at 8192, H = 4096)
    hipLaunchKernelGGL((k_rmsnorm_fwd<T, NV, false, true>), dim3(static_cast<unsigned>(kFwdPipeBlocks1)), dim3(256),
                       0, s, static_cast<const T*>(x), nullptr, static_cast<const T*>(w), nullptr,
                       static_cast<T*>(y), rstd, rows, cols, eps);
  } else {
    hipLaunchKernelGGL((k_rmsnorm_fwd<T, NV, false, false>), dim3(static_cast<unsigned>(need)), dim3(256), 0, s,
                       static_cast<const T*>(x), nullptr, static_cast<const T*>(w), nullptr,
                       static_cast<T*>(y), rstd, rows, cols, eps);
  }
}

// Backward row split: WPR waves per row, NVW chunks of 8 per lane, NWB waves
// per block (RPB = NWB / WPR rows per block step), PF: next-row prefetch.
// Rows of 1025-2048 columns with the residual gradient (the layer's two
// norms) take two waves each in blocks of 8: twice the waves in flight at the
// same partial-row count, 60 -> 56 us at T = 16384, H = 2048 (one wave per
// row in blocks of 8 or 16 needs more than the 128 registers of four waves
// per SIMD).  Rows of 2049-4096 columns with the residual gradient take four
// waves each, with the next row prefetched: kernel time 37.7 -> 33.7 us at
// T = 4096, 60.1 -> 53.8 us at 8192, 206.9 -> 191.6 us at 32768 (H = 4096).
template <int NV, bool RES>
struct BwdSplit {
  static constexpr bool kWide = NV == 8 && RES;
  static constexpr int WPR = kWide ? 4 : NV > 4 || (NV == 4 && RES) ? 2 : 1;
  static constexpr int NVW = NV / WPR;
  static constexpr int NWB = kWide || (NV == 4 && RES) ? 8 : 4;
  static constexpr int RPB = NWB / WPR;
  static constexpr bool PF = !RES || kWide;
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
  hipLaunchKernelGGL((k_rmsnorm_bwd<T, SP::NVW, SP::WPR, SP::NWB, RES, HR, SP::PF>), dim3(blocks), dim3(64 * SP::NWB),
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
  hipLaunchKernelGGL((k_reduce_parts<T>), dim3((cols + 15) / 16), dim3(256), 0, s, part, blocks, cols,
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
  // columns)
  const int64_t nrows = bwd_blocks(rows, cols > 2048 ? 2 : 4);
  return static_cast<size_t>(nrows) * static_cast<size_t>(cols) * sizeof(float);
}

namespace fh {
namespace {

// Scratch of the allocation-free backward: the fp32 partial rows of the
// largest valid call (kMaxBwdBlocks partial rows of at most 8192 columns),
// 16.8 MB per device, held until the process ends.
constexpr size_t kNoAllocScratchFloats = static_cast<size_t>(kMaxBwdBlocks) * 8192;
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
                 (dres == nullptr || aligned16(dres)) && aligned16(workspace),
             "rmsnorm_bwd: pointers (workspace included) must be 16-byte aligned");
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
