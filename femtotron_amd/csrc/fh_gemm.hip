// The projections' GEMMs: C[m, n] = sum_k op(A)[m, k] * op(B)[k, n], bf16 in,
// fp32 accumulation, bf16 out rounded once (optionally plus a residual, rounded
// again, as the layer's residual add does).
//
// Replaces the F.linear of every projection of the layer
// (femtotron/parallel/tensor_parallel/linear.py:66-80, 194-214 at one rank)
// in its three layouts:
//   NT  C = A B^T  (A [M, K], B [N, K])  forward / recompute: x W^T
//   NN  C = A B    (A [M, K], B [K, N])  input gradient:     dY W
//   TN  C = A^T B  (A [K, M], B [K, N])  weight gradient:    dY^T X
// All operands are row-major with a leading dimension (elements).
//
// Block tile 256 (m) x 256 (n), stages of 64 k.  Operand stages go straight
// from global memory into LDS (global_load_lds_dwordx4, two stages of 64 KB:
// A and B, 32 KB each); every load covers whole 128-byte lines (half-line
// requests cost a full line's L2 and DRAM throughput).  Tiles are
// XOR-swizzled so that both read patterns below are free of bank conflicts:
//   * an operand with K contiguous ("KC": A of NT/NN, B of NT) is stored as
//     its [256 x 64] tile; a fragment is one ds_read_b128 per lane (row i%32,
//     k 8*(i/32)..+7);
//   * an operand with K as the outer index ("KO": B of NN, both of TN) is
//     stored as four [64 k x 64] sub-tiles; a fragment is two
//     ds_read_b64_tr_b16 transposing reads that deliver the same natural K
//     order, so any two operands can be paired.
// Eight waves, two per SIMD, each own a 128 (m) x 64 (n) part of the tile (8
// accumulators of v_mfma_f32_32x32x16_bf16).  The two waves of a SIMD take
// turns ("ping-pong"): while one multiplies 32 k of a stage out of registers,
// the other reads its fragments of the next 32 k from LDS and issues the
// global loads of the next stage; a workgroup barrier ends each half-period.
// Waves 4-7 start one half-period late.
//
// The MFMA is issued as (B fragment, A fragment), so accumulator rows run
// along n (C's contiguous index) and every lane stores 4 consecutive outputs.
//
// Few output tiles (a weight gradient of 2048 x 2048 has 64) would leave most
// of the 256 CUs idle, so the K range can be split into S slices whose fp32
// partial tiles are summed in slice order by k_gemm_reduce (deterministic).
#include "fh_common.hpp"
#include "fh_mfma.hpp"

namespace fh {
namespace {

constexpr int kThreads = 512;                  // 8 waves
constexpr int kTm = 256, kTn = 256, kTk = 64;  // block tile and stage depth
constexpr int kOpBytes = 256 * kTk * 2;        // one operand's stage: 32 KB
constexpr int kSubBytes = kTk * 128;           // KO sub-tile: [64 k x 64] bf16

enum Epi { EPI_STORE = 0, EPI_RESIDUAL = 1, EPI_PARTIAL = 2 };

struct GemmArgs {
  const uint16_t* a;
  const uint16_t* b;
  uint16_t* c;
  const uint16_t* r;  // residual (EPI_RESIDUAL)
  float* part;        // fp32 slice partials (EPI_PARTIAL)
  int64_t lda, ldb, ldc, ldr;
  int m, n;
  int tiles_m, tiles_n, tiles;
  int steps_per_slice, total_steps;
  int grid;  // logical blocks (tiles * slices)
};

// Lane offset of a transposing fragment read with K in natural order: lane i
// gets rows 8*(i/32) + plus4 + 0..3 of column i%32 of a 32-wide column block
// of a swizzled [16 x 64] row group (128-byte rows, swz<64>).  The 16 lanes of
// each quarter-wave read one 4-row x 16-column block, lane L 8 bytes of row L/4.
__device__ __forceinline__ int lane_off_tr(int lane, int plus4) {
  const int hl = lane >> 5, L = lane & 15, mh = (lane >> 4) & 1;
  const int r = 8 * hl + (L >> 2) + plus4;
  const int cb = 2 * mh + ((L & 3) >> 1);
  return r * 128 + ((cb ^ swz<64>(r)) << 4) + 8 * (L & 1);
}

// KC fragment: rows o..o+31 of the [256 x 64] tile, k 16*ks + 8*(lane/32) .. +7.
__device__ __forceinline__ bf16x8 frag_kc(const char* tile, int a_off, int o, int ks) {
  return *reinterpret_cast<const bf16x8*>(tile + o * 128 + (a_off ^ (32 * ks)));
}

// KO fragment: columns o..o+31 of the four [64 k x 64] sub-tiles, same k.
__device__ __forceinline__ bf16x8 frag_ko(const char* tile, int t0, int t4, int o, int ks) {
  const char* t = tile + (o >> 6) * kSubBytes + ks * 16 * 128;
  const int x = 64 * ((o >> 5) & 1);
  const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(t + (t0 ^ x)));
  const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(t + (t4 ^ x)));
  const uint2 ulo = __builtin_bit_cast(uint2, lo), uhi = __builtin_bit_cast(uint2, hi);
  return as_bf16x8(make_uint4(ulo.x, ulo.y, uhi.x, uhi.y));
}

// Global -> LDS copy of one wave's quarter (8 runs of 1 KB) of an operand's
// stage.  KC: tile rows 64q .. 64q+63 (clamped to `last`), k0 .. k0+63.  KO:
// sub-tile q, i.e. k rows k0 .. k0+63, columns o0 + 64q .. +63 (chunks
// clamped to `last`, the last 8-column chunk start).  Run jj covers 8 rows of
// 128 bytes; lane i fills 16-byte slot i%8 of row i/8, i.e. it loads the
// chunk the swizzle puts there.  Each address is a wave-uniform 64-bit base
// (clamped too, so the lane offset is never negative) plus a 32-bit lane
// offset (leading dims < 2^26 keep it in range).
template <bool KO>
__device__ __forceinline__ void dma_quarter(const uint16_t* base, int64_t ld, int o0, int last,
                                            int k0, int q, char* dst, int lane) {
  typedef __attribute__((address_space(1))) const void* gptr;
  typedef __attribute__((address_space(3))) void* lptr;
  const int lr = lane >> 3;
#pragma unroll
  for (int jj = 0; jj < 8; ++jj) {
    const int c = (lane & 7) ^ swz<64>(8 * jj + lr);
    const char* sp;
    uint32_t off;
    if constexpr (KO) {
      const int col0 = min(o0 + 64 * q, last);
      sp = reinterpret_cast<const char*>(base + static_cast<int64_t>(k0 + 8 * jj) * ld + col0);
      off = static_cast<uint32_t>(lr * static_cast<int>(ld) + min(o0 + 64 * q + 8 * c, last) - col0) * 2u;
    } else {
      const int row0 = min(o0 + 64 * q + 8 * jj, last);
      sp = reinterpret_cast<const char*>(base + static_cast<int64_t>(row0) * ld + k0);
      off = static_cast<uint32_t>((min(o0 + 64 * q + 8 * jj + lr, last) - row0) * static_cast<int>(ld) +
                                  8 * c) * 2u;
    }
    __builtin_amdgcn_global_load_lds((gptr)(sp + off), (lptr)(dst + (8 * q + jj) * 1024), 16, 0, 0);
  }
}

__device__ __forceinline__ void wait_lds() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
__device__ __forceinline__ void wait_vm() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Workgroup barrier that waits for nothing itself (callers wait first), with
// scheduling fences so no instruction crosses it.
__device__ __forceinline__ void bar() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_barrier" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

template <bool A_KO, bool B_KO, int EPI>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2))) void k_gemm(GemmArgs g) {
  // The two stages as separate arrays (A at 0, B at 32 KB): the loop is
  // unrolled over them, so every LDS access names its stage and the compiler
  // can tell the reads of one stage from the direct-to-LDS loads in flight
  // into the other.
  __shared__ __align__(16) char st0[2 * kOpBytes], st1[2 * kOpBytes];
  const int tid = threadIdx.x, lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2;  // 0: waves 0-3, 1: waves 4-7 (one of each per SIMD)

  // Workgroup L runs on XCD L % 8 (each XCD has its own L2): logical block
  // (L % 8) * (grid / 8) + L / 8 gives every XCD a contiguous run of the
  // logical order below.  The grid is padded to a multiple of 8.
  const int nb8 = gridDim.x >> 3;
  const int lid = (blockIdx.x & 7) * nb8 + (blockIdx.x >> 3);
  if (lid >= g.grid) return;
  const int slice = lid / g.tiles, t = lid - slice * g.tiles;
  // Logical order inside a slice: groups of 4 m tiles, m fastest, so the
  // ~32 tiles an XCD runs at once cover 4 m tiles x 8 n tiles.
  constexpr int GM = 4;
  const int width = GM * g.tiles_n;
  const int gi = t / width, first_m = gi * GM;
  const int gm = min(g.tiles_m - first_m, GM);
  const int tw = t - gi * width;
  const int tm = first_m + tw % gm, tn = tw / gm;
  const int m0 = tm * kTm, n0 = tn * kTn;
  const int s_begin = slice * g.steps_per_slice;
  const int nst = min(g.total_steps - s_begin, g.steps_per_slice);

  // Loads: waves 0-3 copy quarter (wave & 3) of A, waves 4-7 of B.
  const int q = wave & 3;
  auto load = [&](int step, char* stage) __attribute__((always_inline)) {
    const int k0 = (s_begin + step) * kTk;
    if (grp == 0) {
      if constexpr (A_KO) dma_quarter<true>(g.a, g.lda, m0, g.m - 8, k0, q, stage, lane);
      else dma_quarter<false>(g.a, g.lda, m0, g.m - 1, k0, q, stage, lane);
    } else {
      if constexpr (B_KO) dma_quarter<true>(g.b, g.ldb, n0, g.n - 8, k0, q, stage + kOpBytes, lane);
      else dma_quarter<false>(g.b, g.ldb, n0, g.n - 1, k0, q, stage + kOpBytes, lane);
    }
  };

  // Wave tile: m 128*wm .. +127, n 64*wn .. +63.
  const int wm = wave & 1, wn = wave >> 1;
  const int a_off = lane_off_a<64>(lane);
  const int t0 = lane_off_tr(lane, 0), t4 = lane_off_tr(lane, 4);
  bf16x8 fa[2][4], fb[2][2];  // [k16 step of the half][block]
  // Fragments of half h (k 32h .. 32h+31) of a stage.
  auto mem = [&](const char* stage, int h) __attribute__((always_inline)) {
    const char* sa = stage;
    const char* sb = stage + kOpBytes;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int o = 128 * wm + 32 * j;
        fa[ks][j] = A_KO ? frag_ko(sa, t0, t4, o, 2 * h + ks) : frag_kc(sa, a_off, o, 2 * h + ks);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int o = 64 * wn + 32 * i;
        fb[ks][i] = B_KO ? frag_ko(sb, t0, t4, o, 2 * h + ks) : frag_kc(sb, a_off, o, 2 * h + ks);
      }
    }
  };
  f32x16 acc[2][4];  // [n block][m block]; rows = n, column = m
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = zero16();
  // The products of a half; `after_first` runs once the first k16 step's
  // fragments are consumed (their registers are free again).
  auto comp = [&](auto after_first) __attribute__((always_inline)) {
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma(fb[ks][i], fa[ks][j], acc[i][j]);
      if (ks == 0) {
        __builtin_amdgcn_sched_barrier(0);
        after_first();
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    __builtin_amdgcn_s_setprio(0);
  };
  auto nothing = []() __attribute__((always_inline)) {};

  // Half-steps u = 2x + h (stage x, half h).  Phase P(2u): waves 0-3 read half
  // u, waves 4-7 multiply half u-1; phase P(2u+1): the reverse.  Stage x+1 is
  // loaded during P(4x) by all waves, into the stage buffer stage x-1 used
  // (free once P(4x-1) ended), and waited for at the end of P(4x+3), when
  // both groups have read all of stage x.  Every phase ends with a workgroup
  // barrier.
  load(0, st0);
  wait_vm();
  bar();
  if (grp == 0) {
    auto half = [&](int x, int h, const char* cur, char* nxt) __attribute__((always_inline)) {
      if (h == 0 && x + 1 < nst) load(x + 1, nxt);
      mem(cur, h);
      wait_lds();
      bar();
      comp(nothing);
      if (h == 1) wait_vm();
      bar();
    };
    for (int x = 0; x < nst; x += 2) {
      half(x, 0, st0, st1);
      half(x, 1, st0, st1);
      if (x + 1 < nst) {
        half(x + 1, 0, st1, st0);
        half(x + 1, 1, st1, st0);
      }
    }
    bar();  // matches the late start of waves 4-7
  } else {
    if (1 < nst) load(1, st1);
    bar();
    auto half = [&](int x, int h, const char* cur, char* nxt) __attribute__((always_inline)) {
      mem(cur, h);
      wait_lds();
      if (h == 1) wait_vm();
      bar();
      comp([&]() __attribute__((always_inline)) {
        if (h == 1 && x + 2 < nst) load(x + 2, nxt);
      });
      bar();
    };
    for (int x = 0; x < nst; x += 2) {
      half(x, 0, st0, st0);
      half(x, 1, st0, st0);
      if (x + 1 < nst) {
        half(x + 1, 0, st1, st1);
        half(x + 1, 1, st1, st1);
      }
    }
  }

  // lane: m = m0 + 128 wm + 32 j + l32; n = n0 + 64 wn + 32 i + 8 e + 4 hl + 0..3
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int mrow = m0 + 128 * wm + 32 * j + l32;
    if (mrow >= g.m) continue;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int col = n0 + 64 * wn + 32 * i + 8 * e + 4 * hl;
        if (col >= g.n) continue;
        const f32x16& v = acc[i][j];
        if constexpr (EPI == EPI_PARTIAL) {
          float* dst = g.part + (static_cast<int64_t>(slice) * g.m + mrow) * g.n + col;
          *reinterpret_cast<float4*>(dst) = make_float4(v[4 * e], v[4 * e + 1], v[4 * e + 2], v[4 * e + 3]);
        } else if constexpr (EPI == EPI_RESIDUAL) {
          const uint2 rv = *reinterpret_cast<const uint2*>(g.r + mrow * g.ldr + col);
          const float r0 = __uint_as_float(rv.x << 16), r1 = __uint_as_float(rv.x & 0xffff0000u);
          const float r2 = __uint_as_float(rv.y << 16), r3 = __uint_as_float(rv.y & 0xffff0000u);
          *reinterpret_cast<uint2*>(g.c + mrow * g.ldc + col) =
              make_uint2(pk_bf16(r0 + round_bf(v[4 * e]), r1 + round_bf(v[4 * e + 1])),
                         pk_bf16(r2 + round_bf(v[4 * e + 2]), r3 + round_bf(v[4 * e + 3])));
        } else {
          *reinterpret_cast<uint2*>(g.c + mrow * g.ldc + col) =
              make_uint2(pk_bf16(v[4 * e], v[4 * e + 1]), pk_bf16(v[4 * e + 2], v[4 * e + 3]));
        }
      }
  }
}

// C = bf16(sum over slices of part[slice]) (+ residual, rounded as above);
// 4 outputs per thread, slices in order.
template <bool RESID>
__global__ __launch_bounds__(256) void k_gemm_reduce(const float* __restrict__ part, int slices, int m,
                                                     int n, uint16_t* __restrict__ c, int64_t ldc,
                                                     const uint16_t* __restrict__ r, int64_t ldr) {
  const int64_t mn = static_cast<int64_t>(m) * n;
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
  if (i >= mn) return;
  float4 s = *reinterpret_cast<const float4*>(part + i);
  for (int k = 1; k < slices; ++k) {
    const float4 v = *reinterpret_cast<const float4*>(part + static_cast<int64_t>(k) * mn + i);
    s.x += v.x;
    s.y += v.y;
    s.z += v.z;
    s.w += v.w;
  }
  const int64_t row = i / n, col = i - row * n;
  if constexpr (RESID) {
    const uint2 rv = *reinterpret_cast<const uint2*>(r + row * ldr + col);
    s.x = __uint_as_float(rv.x << 16) + round_bf(s.x);
    s.y = __uint_as_float(rv.x & 0xffff0000u) + round_bf(s.y);
    s.z = __uint_as_float(rv.y << 16) + round_bf(s.z);
    s.w = __uint_as_float(rv.y & 0xffff0000u) + round_bf(s.w);
  }
  *reinterpret_cast<uint2*>(c + row * ldc + col) = make_uint2(pk_bf16(s.x, s.y), pk_bf16(s.z, s.w));
}

// Compute units of the current device (one workgroup fits per CU).
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

// K slices S: the modelled time of S slices is ceil(tiles*S / CUs) / S rounds
// of a whole-K tile plus, for S > 1, writing and re-reading the S fp32
// partial outputs (8 bytes per output and slice at ~5 TB/s, against a
// whole-K tile's MFMA time at ~6 TFLOP/s per CU).  Every slice keeps at least
// 256 k.
int gemm_slices(int64_t m, int64_t n, int64_t k) {
  const int64_t tiles = ((m + kTm - 1) / kTm) * ((n + kTn - 1) / kTn), steps = k / kTk;
  const int cus = device_cus();
  const double per_slice = 48.0 * static_cast<double>(m) * n / (655360.0 * static_cast<double>(k));
  int best = 1;
  double best_cost = 1e30;
  for (int s = 1; s <= 8 && s <= k / 256; ++s) {
    const double rounds = static_cast<double>((tiles * s + cus - 1) / cus);
    const double cost = rounds / s + (s > 1 ? per_slice * s : 0.0);
    if (cost < best_cost - 1e-9) {
      best_cost = cost;
      best = s;
    }
  }
  // Slices of ceil(steps / S) stages; fewer if that leaves the last one empty.
  const int64_t per = (steps + best - 1) / best;
  return static_cast<int>((steps + per - 1) / per);
}

template <bool A_KO, bool B_KO>
void launch(const GemmArgs& g, unsigned blocks, bool partial, bool resid, hipStream_t stream) {
  if (partial)
    hipLaunchKernelGGL((k_gemm<A_KO, B_KO, EPI_PARTIAL>), dim3(blocks), dim3(kThreads), 0, stream, g);
  else if (resid)
    hipLaunchKernelGGL((k_gemm<A_KO, B_KO, EPI_RESIDUAL>), dim3(blocks), dim3(kThreads), 0, stream, g);
  else
    hipLaunchKernelGGL((k_gemm<A_KO, B_KO, EPI_STORE>), dim3(blocks), dim3(kThreads), 0, stream, g);
}

bool valid_op(int op) { return op == FH_GEMM_NT || op == FH_GEMM_NN || op == FH_GEMM_TN; }

}  // namespace
}  // namespace fh

using namespace fh;

extern "C" size_t fh_gemm_bf16_workspace_size(int op, int64_t m, int64_t n, int64_t k) {
  if (!valid_op(op) || m <= 0 || n <= 0 || k <= 0 || k % 64) return 0;
  const int s = gemm_slices(m, n, k);
  return s > 1 ? static_cast<size_t>(s) * m * n * sizeof(float) : 0;
}

extern "C" int fh_gemm_bf16(int op, const void* a, int64_t lda, const void* b, int64_t ldb, void* c,
                            int64_t ldc, const void* residual, int64_t ldr, int64_t m, int64_t n,
                            int64_t k, void* workspace, hipStream_t stream) {
  FH_REQUIRE(valid_op(op), "gemm_bf16: op must be FH_GEMM_NT, FH_GEMM_NN or FH_GEMM_TN");
  FH_REQUIRE(m > 0 && n > 0 && k > 0, "gemm_bf16: sizes must be positive");
  FH_REQUIRE(k % 64 == 0, "gemm_bf16: k must be a multiple of 64");
  FH_REQUIRE(n % 8 == 0, "gemm_bf16: n must be a multiple of 8");
  FH_REQUIRE(op != FH_GEMM_TN || m % 8 == 0, "gemm_bf16: m must be a multiple of 8 for FH_GEMM_TN");
  FH_REQUIRE(m < (int64_t(1) << 30) && n < (int64_t(1) << 30) && k < (int64_t(1) << 30),
             "gemm_bf16: sizes too large");
  FH_REQUIRE(lda < (int64_t(1) << 26) && ldb < (int64_t(1) << 26), "gemm_bf16: leading dims >= 2^26");
  // Extents each operand's leading dimension must cover.
  const int64_t a_cols = op == FH_GEMM_TN ? m : k;
  const int64_t b_cols = op == FH_GEMM_NT ? k : n;
  FH_REQUIRE(lda >= a_cols && ldb >= b_cols && ldc >= n && lda % 8 == 0 && ldb % 8 == 0 && ldc % 4 == 0,
             "gemm_bf16: leading dims must cover the rows (a, b multiples of 8, c of 4)");
  FH_REQUIRE(a && b && c, "gemm_bf16: null pointer");
  FH_REQUIRE(aligned16(a) && aligned16(b) && (reinterpret_cast<uintptr_t>(c) & 7u) == 0,
             "gemm_bf16: a and b must be 16-byte aligned, c 8-byte aligned");
  if (residual) {
    FH_REQUIRE(ldr >= n && ldr % 4 == 0 && (reinterpret_cast<uintptr_t>(residual) & 7u) == 0,
               "gemm_bf16: residual must be 8-byte aligned with ldr >= n, a multiple of 4");
    FH_REQUIRE(residual == c ? ldr == ldc : true, "gemm_bf16: residual aliasing c must share its ldc");
  }
  const int slices = gemm_slices(m, n, k);
  FH_REQUIRE(slices == 1 || (workspace && aligned16(workspace)),
             "gemm_bf16: workspace (fh_gemm_bf16_workspace_size bytes) required");

  GemmArgs g;
  g.a = static_cast<const uint16_t*>(a);
  g.b = static_cast<const uint16_t*>(b);
  g.c = static_cast<uint16_t*>(c);
  g.r = static_cast<const uint16_t*>(residual);
  g.part = static_cast<float*>(workspace);
  g.lda = lda;
  g.ldb = ldb;
  g.ldc = ldc;
  g.ldr = ldr;
  g.m = static_cast<int>(m);
  g.n = static_cast<int>(n);
  g.tiles_m = static_cast<int>((m + kTm - 1) / kTm);
  g.tiles_n = static_cast<int>((n + kTn - 1) / kTn);
  g.tiles = g.tiles_m * g.tiles_n;
  g.total_steps = static_cast<int>(k / kTk);
  g.steps_per_slice = (g.total_steps + slices - 1) / slices;
  const int64_t logical = static_cast<int64_t>(g.tiles) * slices;
  FH_REQUIRE(logical <= 0x7ffffff0, "gemm_bf16: grid too large");
  g.grid = static_cast<int>(logical);
  const unsigned blocks = static_cast<unsigned>((logical + 7) / 8 * 8);
  const bool partial = slices > 1, resid = residual != nullptr;
  switch (op) {
    case FH_GEMM_NT: launch<false, false>(g, blocks, partial, resid, stream); break;
    case FH_GEMM_NN: launch<false, true>(g, blocks, partial, resid, stream); break;
    default: launch<true, true>(g, blocks, partial, resid, stream); break;
  }
  if (partial) {
    const int64_t mn = m * n;
    const unsigned rb = static_cast<unsigned>((mn / 4 + 255) / 256);
    if (resid)
      hipLaunchKernelGGL(k_gemm_reduce<true>, dim3(rb), dim3(256), 0, stream, g.part, slices, g.m, g.n, g.c,
                         ldc, g.r, ldr);
    else
      hipLaunchKernelGGL(k_gemm_reduce<false>, dim3(rb), dim3(256), 0, stream, g.part, slices, g.m, g.n,
                         g.c, ldc, nullptr, int64_t(0));
  }
  return check_launch("fh_gemm_bf16");
}
