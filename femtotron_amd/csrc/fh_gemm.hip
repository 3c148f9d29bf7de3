// Weight-gradient GEMM of the projections: C[m, n] = sum_t A[t, m] * B[t, n]
// (C = A^T B), bf16 in, fp32 accumulation, bf16 out rounded once.
//
// Replaces the weight gradient of every projection's F.linear in the layer
// backward (femtotron/parallel/tensor_parallel/linear.py:72, 206 at one rank;
// torch computes grad_weight = grad_output^T @ input): A = the gradient at the
// projection's output [tokens, out_features], B = its input [tokens,
// in_features], both token-major, so the reduction (token) index is the outer
// index of both operands.
//
// Tiles: a 256 x 256 block of C per workgroup of 16 waves (4 per SIMD, so
// memory latency is hidden across waves); each wave holds 64 (m) x 64 (n) as
// 2 x 2 MFMA 32x32 accumulators.  Stages of 64 tokens of
// A and B go through LDS (double-buffered, loaded straight into it with
// global_load_lds: stage s + 1 is in flight while stage s is multiplied), each
// 256-wide operand stored as four swizzled [64 x 64] sub-tiles.  Both MFMA
// operands have K (the token) down the tile rows and are read with
// ds_read_b64_tr_b16 transpose reads in the same permuted K order, so their
// products pair the same tokens.  The accumulator is laid out with rows = n
// (C's contiguous index), so each lane stores 4 consecutive outputs at once.
//
// Few output tiles (a 2048 x 2048 weight has 64) would leave most of the 256
// CUs idle, so the token range is split into S slices (fp32 partial tiles in a
// workspace, summed in slice order by k_gemm_tn_reduce: deterministic).
#include "fh_common.hpp"
#include "fh_mfma.hpp"

namespace fh {
namespace {

constexpr int kGemmThreads = 1024;
constexpr int kTm = 256, kTn = 256, kTk = 64;  // block tile (m, n) and stage depth (tokens)
constexpr int kSub = 64;                       // sub-tile width (swizzled [kTk x 64])
constexpr int kSubBytes = kTk * 2 * kSub;      // 8 KB
constexpr int kStageBytes = 2 * (kTm / kSub) * kSubBytes;  // A and B: 64 KB

template <bool PARTIAL>
__global__ __launch_bounds__(kGemmThreads) __attribute__((amdgpu_waves_per_eu(4))) void k_gemm_tn(
    const uint16_t* __restrict__ a, int64_t lda, const uint16_t* __restrict__ b, int64_t ldb,
    uint16_t* __restrict__ c, int64_t ldc, float* __restrict__ part, int m, int n,
    int steps_per_slice, int total_steps, int tiles_m, int tiles_n) {
  // Two stages (4 A sub-tiles, then 4 B sub-tiles) as separate arrays: the
  // loop is unrolled by two, so every access names its stage and the
  // compiler can tell the loads into one stage from the reads of the other.
  __shared__ __align__(16) char smem0[kStageBytes], smem1[kStageBytes];
  const int tid = threadIdx.x, lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 3, wn = wave >> 2;  // wave tile: m in [64 wm, +64), n in [64 wn, +64)
  // Workgroup L runs on XCD L % 8 (each XCD has its own L2).  Logical block
  // g = (L % 8) * (grid / 8) + L / 8 gives every XCD one contiguous run of the
  // (slice, m tile, n tile) order, i.e. a few m tiles times all n tiles of a
  // slice, so both operand panels are shared inside one L2.
  const int nb = gridDim.x;
  const int g = nb % 8 == 0 ? (blockIdx.x & 7) * (nb >> 3) + (blockIdx.x >> 3) : blockIdx.x;
  const int tiles = tiles_m * tiles_n;
  const int slice = g / tiles, tile = g - slice * tiles;
  const int tm = tile / tiles_n, tn = tile - tm * tiles_n;
  const int m0 = tm * kTm, n0 = tn * kTn;
  const int s_begin = slice * steps_per_slice;
  const int s_end = min(total_steps, s_begin + steps_per_slice);
  int b0 = lane_off_b<kSub>(lane, 0), b8 = lane_off_b<kSub>(lane, 8);

  // Loads: wave w fills sub-tile w / 2 of a stage (A: 0-3, B: 4-7), half of
  // its eight 1 KB runs each (dma_tile with two waves per sub-tile).
  const int lsub = wave >> 1;
  const bool op_b = lsub >= kTm / kSub;
  const uint16_t* src = (op_b ? b + n0 : a + m0) + (lsub & 3) * kSub;
  const int64_t ld = op_b ? ldb : lda;
  const int lds_dst = lsub * kSubBytes;
  const int last_row = total_steps * kTk - 1;
  auto load = [&](int step, char* stage) __attribute__((always_inline)) {
    dma_tile<kTk, kSub, 2>(src, ld, step * kTk, last_row, stage + lds_dst, wave & 1, lane);
  };

  f32x16 acc[2][2];  // [n block][m block], rows = n, column = m
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = zero16();

  if (s_begin < s_end) load(s_begin, smem0);
  wait_loads();
  __syncthreads();
  // Stage `step` from `cur` while stage step + 1 is loaded into `nxt`.
  auto step_fn = [&](int step, const char* cur, char* nxt) __attribute__((always_inline)) {
    asm volatile("" : "+v"(b0), "+v"(b8));  // keep the XORed read offsets recomputed
    if (step + 1 < s_end) load(step + 1, nxt);
    if (step < s_end) {
      const char* sa = cur;
      const char* sb = cur + (kTm / kSub) * kSubBytes;
#pragma unroll
      for (int ks = 0; ks < kTk / 16; ++ks) {
        bf16x8 fa[2], fb[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {  // the wave's 64 m are sub-tile wm; its 64 n sub-tile wn
          fa[i] = lds_frag_tr<kSub>(sa + wm * kSubBytes, b0, b8, 16 * ks, i);
          fb[i] = lds_frag_tr<kSub>(sb + wn * kSubBytes, b0, b8, 16 * ks, i);
        }
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j) acc[i][j] = mfma(fb[i], fa[j], acc[i][j]);
      }
    }
    wait_loads();
    __syncthreads();
  };
  for (int step = s_begin; step < s_end; step += 2) {
    step_fn(step, smem0, smem1);
    step_fn(step + 1, smem1, smem0);
  }

  // lane: column m = m0 + 64 wm + 32 j + l32; rows n = n0 + 64 wn + 32 i + 8 g + 4 hl + 0..3
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int64_t mrow = m0 + 64 * wm + 32 * j + l32;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int col = n0 + 64 * wn + 32 * i + 8 * g + 4 * hl;
        const f32x16& v = acc[i][j];
        if constexpr (PARTIAL) {
          float* dst = part + (static_cast<int64_t>(slice) * m + mrow) * n + col;
          *reinterpret_cast<float4*>(dst) = make_float4(v[4 * g], v[4 * g + 1], v[4 * g + 2], v[4 * g + 3]);
        } else {
          *reinterpret_cast<uint2*>(c + mrow * ldc + col) =
              make_uint2(pk_bf16(v[4 * g], v[4 * g + 1]), pk_bf16(v[4 * g + 2], v[4 * g + 3]));
        }
      }
  }
}

// C = bf16(sum over slices of part[slice]), 8 outputs per thread, slices in order.
__global__ __launch_bounds__(256) void k_gemm_tn_reduce(const float* __restrict__ part, int slices,
                                                        int64_t mn, int n, uint16_t* __restrict__ c,
                                                        int64_t ldc) {
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 8;
  if (i >= mn) return;
  float s[8];
  Elem<float>::load8(part + i, s);
  for (int k = 1; k < slices; ++k) {
    float v[8];
    Elem<float>::load8(part + static_cast<int64_t>(k) * mn + i, v);
#pragma unroll
    for (int e = 0; e < 8; ++e) s[e] += v[e];
  }
  const int64_t row = i / n, col = i - row * n;
  Elem<uint16_t>::store8(c + row * ldc + col, s);
}

// Compute units of the current device (one 128 KB-LDS workgroup fits per CU).
int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      cus = 256;
    cached[dev] = cus;
  }
  return cached[dev];
}

// Token slices S: the modelled time of S slices is ceil(tiles*S / CUs) / S
// rounds of a whole-range tile (each workgroup does 1/S of the tokens) plus,
// for S > 1, writing and re-reading S fp32 partial outputs (8 bytes per
// output and slice at ~5 TB/s against a tile's MFMA time at ~6 TFLOP/s per CU).
// Every slice keeps at least 4 stages.
int gemm_slices(int64_t m, int64_t n, int64_t k) {
  const int64_t tiles = (m / kTm) * (n / kTn), steps = k / kTk;
  const int cus = device_cus();
  const double per_slice = 48.0 * static_cast<double>(m) * n / (655360.0 * static_cast<double>(k));
  int best = 1;
  double best_cost = 1e30;
  for (int s = 1; s <= 8 && s <= steps / 4; ++s) {
    const double waves = static_cast<double>((tiles * s + cus - 1) / cus);
    const double cost = waves / s + (s > 1 ? per_slice * s : 0.0);
    if (cost < best_cost - 1e-9) {
      best_cost = cost;
      best = s;
    }
  }
  return best;
}

}  // namespace
}  // namespace fh

using namespace fh;

extern "C" size_t fh_gemm_tn_workspace_size(int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || n <= 0 || k <= 0 || m % kTm || n % kTn || k % kTk) return 0;
  const int s = gemm_slices(m, n, k);
  return s > 1 ? static_cast<size_t>(s) * m * n * sizeof(float) : 0;
}

extern "C" int fh_gemm_tn(fh_dtype dt, const void* a, int64_t lda, const void* b, int64_t ldb, void* c,
                          int64_t ldc, int64_t m, int64_t n, int64_t k, void* workspace,
                          hipStream_t stream) {
  FH_REQUIRE(dt == FH_BF16, "gemm_tn: dtype must be FH_BF16");
  FH_REQUIRE(m > 0 && n > 0 && k > 0, "gemm_tn: sizes must be positive");
  FH_REQUIRE(m % kTm == 0 && n % kTn == 0 && k % kTk == 0,
             "gemm_tn: m and n must be multiples of 256 and k a multiple of 64");
  FH_REQUIRE(m < (int64_t(1) << 30) && n < (int64_t(1) << 30) && k < (int64_t(1) << 31),
             "gemm_tn: sizes too large");
  FH_REQUIRE(lda >= m && ldb >= n && ldc >= n && lda % 8 == 0 && ldb % 8 == 0 && ldc % 8 == 0,
             "gemm_tn: leading dims must cover the rows and be multiples of 8");
  FH_REQUIRE(a && b && c, "gemm_tn: null pointer");
  FH_REQUIRE(aligned16(a) && aligned16(b) && aligned16(c), "gemm_tn: pointers must be 16-byte aligned");
  const int slices = gemm_slices(m, n, k);
  FH_REQUIRE(slices == 1 || (workspace && aligned16(workspace)),
             "gemm_tn: workspace (fh_gemm_tn_workspace_size bytes) required");
  const int tiles_m = static_cast<int>(m / kTm), tiles_n = static_cast<int>(n / kTn);
  const int total = static_cast<int>(k / kTk);
  const int per = (total + slices - 1) / slices;
  const int64_t blocks = static_cast<int64_t>(tiles_m) * tiles_n * slices;
  FH_REQUIRE(blocks <= 0x7fffffff, "gemm_tn: grid too large");
  const auto* pa = static_cast<const uint16_t*>(a);
  const auto* pb = static_cast<const uint16_t*>(b);
  auto* pc = static_cast<uint16_t*>(c);
  if (slices == 1) {
    hipLaunchKernelGGL(k_gemm_tn<false>, dim3(static_cast<unsigned>(blocks)), dim3(kGemmThreads), 0,
                       stream, pa, lda, pb, ldb, pc, ldc, nullptr, static_cast<int>(m),
                       static_cast<int>(n), per, total, tiles_m, tiles_n);
  } else {
    float* part = static_cast<float*>(workspace);
    hipLaunchKernelGGL(k_gemm_tn<true>, dim3(static_cast<unsigned>(blocks)), dim3(kGemmThreads), 0,
                       stream, pa, lda, pb, ldb, pc, ldc, part, static_cast<int>(m), static_cast<int>(n),
                       per, total, tiles_m, tiles_n);
    const int64_t mn = m * n;
    hipLaunchKernelGGL(k_gemm_tn_reduce, dim3(static_cast<unsigned>((mn / 8 + 255) / 256)), dim3(256), 0,
                       stream, part, slices, mn, static_cast<int>(n), pc, ldc);
  }
  return check_launch("fh_gemm_tn");
}
