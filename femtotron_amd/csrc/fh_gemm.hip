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
// Block tile 256 (m) x 256 (n), stages of 64 k, four waves (one per SIMD),
// each owning a 128 x 128 part of the tile in 64 AGPR accumulators of
// v_mfma_f32_16x16x32_bf16 (under the power limit this MFMA sustains a ~15%
// higher clock than 32x32x16 at the same work per cycle: 1.93 against 1.75
// PFLOP/s in a stream of independent MFMAs).  Operands go straight from global memory into LDS
// (global_load_lds_dwordx4, 1 KB per instruction; every load covers whole
// 128-byte lines, as half-line requests cost a full line's L2 and DRAM
// throughput).  LDS holds a ring of five operand slots (A or B of one stage,
// 32 KB each: 160 KB), so the loads of stage x+2 can start while stage x is
// multiplied and are spread over its 128 MFMAs: the load instructions issue at
// ~1 KB per 16 cycles per CU, and a burst of them right after a barrier would
// hold up the MFMAs behind it.  Fragments are read from LDS one k32 step ahead
// of the MFMAs that use them.  The two tile layouts keep their read
// patterns free of bank conflicts:
//   * an operand with K contiguous ("KC": A of NT/NN, B of NT) is stored as
//     its [256 x 64] tile; a fragment is one ds_read_b128 per lane (row i%16,
//     k 8*(i/16)..+7 of the k32 step);
//   * an operand with K as the outer index ("KO": B of NN, both of TN) is
//     stored as four [64 k x 64] sub-tiles of eight 1 KB units (8 k rows),
//     each unit four 256-byte blocks of 16 columns (row r's 32 bytes at 32 r:
//     no swizzle); a fragment is two ds_read_b64_tr_b16 transposing reads
//     that deliver the same natural K order, so any two operands can be
//     paired.  A quarter-wave's read covers 128 contiguous bytes (full LDS
//     rate: 4 cycles per read and wave, against 4.8 with the 64-column rows
//     XOR-swizzled), and a fragment's address is one per-lane offset plus
//     immediates.
// The MFMA is issued as (B fragment, A fragment), so each lane's four
// accumulator values are consecutive along n (C's contiguous index).  The finished tile goes through LDS so that
// every global store writes whole rows.
//
// Few output tiles (a weight gradient of 2048 x 2048 has 64) would leave most
// of the 256 CUs idle, so the K range can be split into S slices whose fp32
// partial tiles are summed in slice order by k_gemm_reduce (deterministic).
// Where the tiles leave a last round of CUs partly idle (the gate/up weight
// gradient's 352 tiles: 1.375 rounds), the stream form instead gives every CU
// one workgroup and the same number of k-steps: whole tiles first, then an
// even share of the remaining tiles' k-steps, whose split tiles k_gemm_fixup
// sums from fp32 segments in k order (deterministic, no inter-workgroup
// waits).
#include "fh_common.hpp"
#include "fh_mfma.hpp"

#include <algorithm>
#include <mutex>
#include <type_traits>

namespace fh {
namespace {

#ifndef FH_GEMM_PERSIST
#define FH_GEMM_PERSIST 1  // whole-K GEMMs with plain stores in the persistent form
#endif

constexpr int kTm = 256, kTn = 256, kTk = 64;  // block tile and stage depth
constexpr int kSubBytes = kTk * 128;           // KO sub-tile: [64 k x 64] bf16

enum Epi { EPI_STORE = 0, EPI_RESIDUAL = 1, EPI_PARTIAL = 2, EPI_ROPE = 3, EPI_STREAM = 4 };

// The rotary embedding of EPI_ROPE: columns [0, rot_cols) of C are heads of
// hd columns (hd a power of two dividing the 256-column tile, so no head
// straddles a tile); row t of C is a token at position t % seq_len
// (per_token == 0: cos/sin rows are positions) or t (per_token: rows are
// tokens).
struct GemmRope {
  const uint16_t* cos;
  const uint16_t* sin;
  int rot_cols, hd, per_token, seq_len;
  FastDiv seq;
};

// One problem of a grouped stream GEMM (the same op and k for all): its
// operands and the first of its tiles in the group's tile order.
constexpr int kMaxGroup = 3;
struct GemmProblem {
  const uint16_t* a;
  const uint16_t* b;
  uint16_t* c;
  const uint16_t* r;
  int64_t lda, ldb, ldc, ldr;
  int m, n, tiles_m, tiles_n, tile0;
};

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
  int grid;  // logical blocks (tiles * slices; EPI_STREAM: the workgroups)
  // EPI_STREAM: full_rounds whole tiles per workgroup (tile r * grid + w),
  // then the remaining tail_tiles' tail_iters = tail_tiles * total_steps
  // k-steps split evenly over the workgroups
  int full_rounds, tail_tiles;
  int64_t tail_iters;
  // > 0: the tail in XCD slabs (tail_tiles = slab_chunks * grid / 8; see k_gemm)
  int slab_chunks;
  GemmRope rope;
  // EPI_STREAM: the problems (one, or several of the same op and k that share
  // the launch), tiles numbered problem by problem
  int ngroup;
  GemmProblem grp[kMaxGroup];
};

// Two bf16 sums res + c of packed pairs, each rounded to bf16 (the residual
// add of a bf16 projection output: torch's bf16 + bf16).
__device__ __forceinline__ uint32_t add_bf16x2(uint32_t res, uint32_t c) {
  return pk_bf16(__uint_as_float(res << 16) + __uint_as_float(c << 16),
                 __uint_as_float(res & 0xffff0000u) + __uint_as_float(c & 0xffff0000u));
}

// 8 outputs of the forward rotation (rope_fwd_one) from this chunk x, its
// partner chunk p (hd/2 columns away in the head), and the cos / signed sin
// chunks of its own columns.
__device__ __forceinline__ uint4 rope_fwd_chunk(uint4 x, uint4 p, uint4 c, uint4 s) {
  float xf[8], pf[8], cf[8], sf[8], o[8];
  Elem<uint16_t>::unpack(x, xf);
  Elem<uint16_t>::unpack(p, pf);
  Elem<uint16_t>::unpack(c, cf);
  Elem<uint16_t>::unpack(s, sf);
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = rope_fwd_one<uint16_t>(xf[e], pf[e], cf[e], sf[e]);
  return Elem<uint16_t>::pack(o);
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

// As inline asm with the accumulator tied in place ("+a"): through the
// builtin, the register allocator gave 64 four-register accumulators
// different source and destination tuples and shuffled them through VGPRs
// (~130 extra moves per stage).  The compiler's hazard checks do not see an
// asm MFMA: the kernel pads the two hazards this code has itself (an
// accumulator zeroed just before its first MFMA; MFMA results read right
// after the last one) with s_nop.
__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
  return c;
}

// 16x16x32 KC fragment: lane i reads row i%16, k chunk i/16 of a k32 step
// (chunk 4 ks + i/16 of the row's eight; rows o..o+15 of the [256 x 64] tile,
// o a multiple of 16, share swz<64>, which depends on row bits 1..3 only).
__device__ __forceinline__ int lane_off_kc16(int lane) {
  const int r = lane & 15;
  return r * 128 + (((lane >> 4) ^ swz<64>(r)) << 4);
}

__device__ __forceinline__ bf16x8 frag_kc16(const char* tile, int a_off, int o, int ks) {
  return *reinterpret_cast<const bf16x8*>(tile + o * 128 + (a_off ^ (64 * ks)));
}

// 16x16x32 KO fragment lane offset: quarter-wave q = i/16 reads unit q of the
// k32 step (k rows 8 q .. 8 q + 7) and in it rows plus4 + 0..3 of a 16-column
// block (lane L = i%16: 8 bytes of row L/4, columns 4 (L%4) .. +3), so that
// lane i gets column i%16, k 8 q .. 8 q + 7 over the two reads, as a KC
// fragment holds them.  The reads with plus4 = 4 are 128 bytes further.
__device__ __forceinline__ int lane_off_tr16(int lane) {
  const int q = lane >> 4, L = lane & 15;
  return q * 1024 + (2 * (L >> 2) + ((L & 3) >> 1)) * 16 + 8 * (L & 1);
}

// KO fragment: columns o..o+15 (o a multiple of 16, block (o % 64) / 16 of
// sub-tile o / 64), k rows 32 ks .. 32 ks + 31 (units 4 ks .. 4 ks + 3).
__device__ __forceinline__ bf16x8 frag_ko16(const char* tile, int t0, int o, int ks) {
  const char* t = tile + (o >> 6) * kSubBytes + ks * 4096 + ((o >> 4) & 3) * 256 + t0;
  const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)t);
  const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(t + 128));
  const uint2 ulo = __builtin_bit_cast(uint2, lo), uhi = __builtin_bit_cast(uint2, hi);
  return as_bf16x8(make_uint4(ulo.x, ulo.y, uhi.x, uhi.y));
}

// The loads go through dma16 (fh_mfma.hpp): inline asm, so that the compiler
// does not track them (it would otherwise wait for every load in flight before
// any LDS read); the kernel waits for its loads itself (s_waitcnt vmcnt) before
// the barrier that hands a stage to the other waves.

// Wave q's quarter of one operand's stage is 8 runs jj, each one 1 KB load
// into slot (8q + jj) of the stage's tile.  KC: tile rows 64q + 8jj .. +7
// (clamped to `last`), k0 .. k0+63: lane i fills 16-byte slot i%8 of row i/8,
// i.e. it loads the chunk the swizzle puts there.  KO: unit jj of sub-tile q,
// k rows k0 + 8jj .. +7, columns o0 + 64q .. +63 (chunks clamped to `last`,
// the last 8-column chunk start): lane i fills 16-byte slot i%16 of block
// i/16, i.e. chunk i%2 of that block's 32 bytes of row (i%16)/2.  A load's address is a wave-uniform 64-bit base
// (clamped too, so the lane offset is never negative) plus a 32-bit lane offset
// (leading dims < 2^26 keep it in range).  The plan holds, per tile, each run's
// base without the k offset and the lane offsets, so that a load in the loop
// costs one 64-bit scalar add of the stage's k offset (k0 elements for KC, k0
// rows for KO); recomputing (k0 + 8jj) * ld for every KO load put a 64-bit
// scalar multiply chain in front of each one, ~180 cycles per stage and KO
// operand.  A KO lane offset is the same for every run.
template <bool KO>
struct RunPlan {
  const char* run[8];
  uint32_t off[KO ? 1 : 8];
  int64_t k_bytes;  // bytes per k (KO: a row, ld elements; KC: one element)

  __device__ __forceinline__ void init(const uint16_t* base, int64_t ld, int o0, int last, int q, int lane) {
    if constexpr (KO) {
      const int col0 = min(o0 + 64 * q, last);
#pragma unroll
      for (int jj = 0; jj < 8; ++jj)
        run[jj] = reinterpret_cast<const char*>(base + static_cast<int64_t>(8 * jj) * ld + col0);
      const int r = (lane >> 1) & 7, c = 2 * (lane >> 4) + (lane & 1);
      off[0] = static_cast<uint32_t>(r * static_cast<int>(ld) + min(o0 + 64 * q + 8 * c, last) - col0) * 2u;
      k_bytes = ld * 2;
    } else {
      const int lr = lane >> 3;
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        const int row0 = min(o0 + 64 * q + 8 * jj, last);
        const int c = (lane & 7) ^ swz<64>(8 * jj + lr);
        run[jj] = reinterpret_cast<const char*>(base + static_cast<int64_t>(row0) * ld);
        off[jj] = static_cast<uint32_t>((min(o0 + 64 * q + 8 * jj + lr, last) - row0) * static_cast<int>(ld) + 8 * c) * 2u;
      }
      k_bytes = 2;
    }
  }

  // Run jj of the stage k_off bytes along k (k0 * k_bytes) into the LDS
  // slot at byte address lds_slot.
  __device__ __forceinline__ void load(int64_t k_off, int jj, uint32_t lds_slot) const {
    dma16(off[KO ? 0 : jj], run[jj] + k_off, lds_slot);
  }
  // load() with M0 already holding lds_slot (set_m0 at least one instruction earlier).
  __device__ __forceinline__ void load_m0(int64_t k_off, int jj) const { dma16_m0(off[KO ? 0 : jj], run[jj] + k_off); }
};

__device__ __forceinline__ void wait_lds() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
__device__ __forceinline__ void wait_vm() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Workgroup barrier that waits for nothing itself (callers wait first), with
// scheduling fences so no instruction crosses it.
__device__ __forceinline__ void bar() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_barrier" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

constexpr int kSlot = 32768;  // one operand's stage: [256 x 64] bf16
constexpr int kRing = 5;      // operand slots in LDS (160 KB)

template <int N>
__device__ __forceinline__ void wait_vm_n() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ int mod5(int v) { return v >= 5 ? v - 5 : v; }

// Origin of tile t: tiles run in groups of GM = 4 m-tiles, n-major inside a
// group, so consecutive tiles (and the workgroups of one XCD) share B columns
// and A rows in L2.
__device__ __forceinline__ void tile_origin(const GemmArgs& g, int t, int& m0, int& n0) {
  constexpr int GM = 4;
  const int width = GM * g.tiles_n;
  const int gi = t / width, first_m = gi * GM;
  const int gm = min(g.tiles_m - first_m, GM);
  const int tw = t - gi * width;
  m0 = (first_m + tw % gm) * kTm;
  n0 = (tw / gm) * kTn;
}

// The arguments of the problem that holds tile t of a stream GEMM's tile
// order, with t made local to it (the group table holds every stream GEMM's
// problems, one or more).
__device__ __forceinline__ GemmArgs for_tile(const GemmArgs& g, int& t) {
  int p = 0;
#pragma unroll
  for (int i = 1; i < kMaxGroup; ++i) p = (i < g.ngroup && t >= g.grp[i].tile0) ? i : p;
  const GemmProblem& P = g.grp[p];
  GemmArgs q = g;
  q.a = P.a;
  q.b = P.b;
  q.c = P.c;
  q.r = P.r;
  q.lda = P.lda;
  q.ldb = P.ldb;
  q.ldc = P.ldc;
  q.ldr = P.ldr;
  q.m = P.m;
  q.n = P.n;
  q.tiles_m = P.tiles_m;
  q.tiles_n = P.tiles_n;
  t -= P.tile0;
  return q;
}

// One tile t over k-steps s_begin .. s_begin + nst - 1.  The result goes to C
// (bf16, with the EPI epilogue) or, for EPI_PARTIAL and for EPI_STREAM with
// to_part, as fp32 to pdst (the tile's origin, row stride pld).  EPI_STREAM
// ends with a barrier, as the workgroup's next tile reuses the LDS ring.
template <bool A_KO, bool B_KO, int EPI>
__device__ __forceinline__ void gemm_tile(const GemmArgs& g, char* ring, int t, int s_begin, int nst,
                                          float* pdst, int64_t pld, bool to_part) {
  const int tid = threadIdx.x, lane = tid & 63, hl = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  int m0, n0;
  tile_origin(g, t, m0, n0);

  RunPlan<A_KO> pa;
  RunPlan<B_KO> pb;
  pa.init(g.a, g.lda, m0, A_KO ? g.m - 8 : g.m - 1, wave, lane);
  pb.init(g.b, g.ldb, n0, B_KO ? g.n - 8 : g.n - 1, wave, lane);
  typedef __attribute__((address_space(3))) char* lptr;
  const uint32_t ring0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lptr)ring)) + wave * 8192;

  // Run jj of wave `wave`'s quarter of operand OP (0: A, 1: B) of stage
  // `step` into ring slot `slot`.  Stages past the slice's end re-load its
  // last stage (in bounds, never used): the loop has no branches.
  auto dma = [&](auto op_tag, int step, int slot, int jj) __attribute__((always_inline)) {
    constexpr int OP = decltype(op_tag)::value;
    const int64_t k0 = static_cast<int64_t>(s_begin + min(step, nst - 1)) * kTk;
    const uint32_t lds_slot = ring0 + slot * kSlot + jj * 1024;
    if constexpr (OP == 0) pa.load(k0 * pa.k_bytes, jj, lds_slot);
    else pb.load(k0 * pb.k_bytes, jj, lds_slot);
  };
  // The loop's form: M0 set one MFMA earlier (set_m0), so the load needs no s_nop.
  auto dma_m0 = [&](auto op_tag, int step, int jj) __attribute__((always_inline)) {
    constexpr int OP = decltype(op_tag)::value;
    const int64_t k0 = static_cast<int64_t>(s_begin + min(step, nst - 1)) * kTk;
    if constexpr (OP == 0) pa.load_m0(k0 * pa.k_bytes, jj);
    else pb.load_m0(k0 * pb.k_bytes, jj);
  };
  using OpA = std::integral_constant<int, 0>;
  using OpB = std::integral_constant<int, 1>;

  const int wm = wave & 1, wn = wave >> 1;
  // v_mfma_f32_16x16x32_bf16: the wave's 128 x 128 outputs are 8 (n) x 8 (m)
  // accumulators of 16 x 16; a stage is two k32 steps of 64 MFMAs.  Operand
  // lane i holds row/column i%16 and k 8*(i/16) .. +7 of the step.
  const int a_off = lane_off_kc16(lane);
  const int t0 = lane_off_tr16(lane);
  bf16x8 fa[2][8], fb[2][8];
  // Fragment r = 0..15 of k32 step ks (order B0, A0..A7, B1..B7: the order
  // the MFMAs first use them) from slots sa (A) and sb (B).
  auto rd1 = [&](int sa, int sb, int ks, int buf, int r) __attribute__((always_inline)) {
    if (r >= 1 && r <= 8) {
      const char* tile = ring + sa * kSlot;
      const int j = r - 1, o = 128 * wm + 16 * j;
      fa[buf][j] = A_KO ? frag_ko16(tile, t0, o, ks) : frag_kc16(tile, a_off, o, ks);
    } else {
      const char* tile = ring + sb * kSlot;
      const int i = r == 0 ? 0 : r - 8, o = 128 * wn + 16 * i;
      fb[buf][i] = B_KO ? frag_ko16(tile, t0, o, ks) : frag_kc16(tile, a_off, o, ks);
    }
  };
  f32x4 acc[8][8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto mf1 = [&](int buf, int nn) __attribute__((always_inline)) {
    const int i = nn >> 3, j = nn & 7;
    acc[i][j] = mfma16(fb[buf][i], fa[buf][j], acc[i][j]);
  };

  // Operand u (A of stage x: u = 2x, B: 2x+1) lives in ring slot u % 5.
  // Prologue: stages 0 and 1, wait for stage 0, read its step-0 fragments.
#pragma unroll
  for (int jj = 0; jj < 8; ++jj) dma(OpA(), 0, 0, jj);
#pragma unroll
  for (int jj = 0; jj < 8; ++jj) dma(OpB(), 0, 1, jj);
#pragma unroll
  for (int jj = 0; jj < 8; ++jj) dma(OpA(), 1, 2, jj);
#pragma unroll
  for (int jj = 0; jj < 8; ++jj) dma(OpB(), 1, 3, jj);
  wait_vm_n<16>();
  bar();
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    rd1(0, 1, 0, 0, r);
    __builtin_amdgcn_sched_barrier(0);
  }

  // Stage x (A in slot s, B in s+1; stage x+1 in s+2, s+3; s+4 free):
  //   step 0: 64 MFMAs on buffer 0 while step 1's fragments are read into
  //     buffer 1 (one read per 4 MFMAs) and A(x+2) is loaded into s+4;
  //   then each wave waits for its reads and for every load but A(x+2)'s
  //   (stage x+1 complete in LDS), and the barrier: stage x's slots are
  //   read no more;
  //   step 1: 64 MFMAs on buffer 1 while the next stage's step-0 fragments
  //     are read into buffer 0 and B(x+2) is loaded into slot s.
  int s = 0;
  for (int x = 0; x < nst; ++x) {
    const int sB = mod5(s + 1), nA = mod5(s + 2), nB = mod5(s + 3), fA = mod5(s + 4);
    // VALU writes of an accumulator (the zeroing before the loop) need wait
    // states before an MFMA reads it.
    asm volatile("s_nop 4");
#pragma unroll
    for (int p = 0; p < 64; ++p) {
      if ((p & 3) == 0) rd1(s, sB, 1, 1, p >> 2);
      if ((p & 7) == 1) set_m0(ring0 + fA * kSlot + (p >> 3) * 1024);
      if ((p & 7) == 2) dma_m0(OpA(), x + 2, p >> 3);
      mf1(0, p);
      __builtin_amdgcn_sched_barrier(0);
    }
    wait_lds();
    wait_vm_n<8>();
    bar();
#pragma unroll
    for (int p = 0; p < 64; ++p) {
      if ((p & 3) == 0) rd1(nA, nB, 0, 0, p >> 2);
      if ((p & 7) == 1) set_m0(ring0 + s * kSlot + (p >> 3) * 1024);
      if ((p & 7) == 2) dma_m0(OpB(), x + 2, p >> 3);
      mf1(1, p);
      __builtin_amdgcn_sched_barrier(0);
    }
    s = nA;
    // MFMA results need wait states before other instructions read them
    // (at most 18): after the last stage, before anything (the staging
    // below, or a copy the register allocator places at the loop's exit)
    // reads the accumulators.
    if (x == nst - 1) asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7");
  }
  __builtin_amdgcn_sched_barrier(0);
  // The re-loads past the end and the last stale fragment reads complete
  // before the ring is reused for the output tile.
  wait_vm();
  wait_lds();
  bar();

  if (EPI == EPI_PARTIAL || (EPI == EPI_STREAM && to_part)) {
    // The fp32 tile goes through LDS in two halves of 128 rows ([128 rows x
    // 256 columns], 16-byte chunk c of row r stored at chunk c ^ (r % 16));
    // lane i of a wave then stores chunk i of a 1 KB row.
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      if (wm == half) {
        // lane i of accumulator (i, j): row 16 j + i%16, columns
        // 128 wn + 16 i + 4 (i/16) .. +3 (one 16-byte chunk)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int r = 16 * j + (lane & 15);
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const int chunk = 32 * wn + 4 * i + (lane >> 4);
            const f32x4& v = acc[i][j];
            *reinterpret_cast<float4*>(ring + r * 1024 + ((chunk ^ (r & 15)) << 4)) =
                make_float4(v[0], v[1], v[2], v[3]);
          }
        }
      }
      wait_lds();
      bar();
      const int col = n0 + 4 * lane;
#pragma unroll 4
      for (int q2 = 0; q2 < 32; ++q2) {
        const int r = 32 * wave + q2;
        const float4 v = *reinterpret_cast<const float4*>(ring + r * 1024 + ((lane ^ (r & 15)) << 4));
        const int mrow = m0 + 128 * half + r;
        if (mrow < g.m && col < g.n)
          *reinterpret_cast<float4*>(pdst + static_cast<int64_t>(128 * half + r) * pld + 4 * lane) = v;
      }
      wait_lds();
      bar();
    }
  } else {
    // The bf16 tile goes through LDS ([256 rows x 256 columns], 16-byte chunk
    // c of row r stored at chunk c ^ (r % 16)) so that every global store
    // writes whole rows: lane i of a wave stores chunk i % 32 of row 2q + i / 32.
    // lane i of accumulator (i, j): row 128 wm + 16 j + i%16, columns
    // 128 wn + 16 i + 4 (i/16) .. +3 (half a 16-byte chunk)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int r = 128 * wm + 16 * j + (lane & 15);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int chunk = 16 * wn + 2 * i + (lane >> 5);
        const f32x4& v = acc[i][j];
        *reinterpret_cast<uint2*>(ring + r * 512 + ((chunk ^ (r & 15)) << 4) + 8 * ((lane >> 4) & 1)) =
            make_uint2(pk_bf16(v[0], v[1]), pk_bf16(v[2], v[3]));
      }
    }
    wait_lds();
    bar();
    const int chunk = lane & 31;
    const int col = n0 + 8 * chunk;
    if constexpr (EPI == EPI_ROPE) {
      // Rotated columns read their partner chunk (hd/2 columns away, same
      // head, same row) from the staged tile and the cos / sin chunks of
      // their own columns; eight rows' loads are issued before their math.
      const GemmRope& rp = g.rope;
      const bool rot = col < rp.rot_cols;
      const int hc = rp.hd >> 4, pc = chunk ^ hc, cofs = col & (rp.hd - 1);
      const uint32_t sflip = (chunk & hc) ? 0u : 0x80008000u;  // lower half of a head: -sin
#pragma unroll 1
      for (int q0 = 0; q0 < 32; q0 += 8) {
        uint4 v[8], pv[8], cv[8], sv[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int r = 64 * wave + 2 * (q0 + u) + hl;
          v[u] = *reinterpret_cast<const uint4*>(ring + r * 512 + ((chunk ^ (r & 15)) << 4));
          if (rot) {
            pv[u] = *reinterpret_cast<const uint4*>(ring + r * 512 + ((pc ^ (r & 15)) << 4));
            const int t = min(m0 + r, g.m - 1);  // rows past m: an in-bounds read, never stored
            const int pos = rp.per_token ? t : t - static_cast<int>(rp.seq.div(static_cast<uint32_t>(t))) * rp.seq_len;
            const int64_t tb = static_cast<int64_t>(pos) * rp.hd + cofs;
            cv[u] = *reinterpret_cast<const uint4*>(rp.cos + tb);
            sv[u] = *reinterpret_cast<const uint4*>(rp.sin + tb);
          }
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int mrow = m0 + 64 * wave + 2 * (q0 + u) + hl;
          uint4 o = v[u];
          if (rot)
            o = rope_fwd_chunk(v[u], pv[u], cv[u],
                               make_uint4(sv[u].x ^ sflip, sv[u].y ^ sflip, sv[u].z ^ sflip, sv[u].w ^ sflip));
          if (mrow < g.m && col < g.n) *reinterpret_cast<uint4*>(g.c + mrow * g.ldc + col) = o;
        }
      }
      return;
    }
#pragma unroll 4
    for (int q2 = 0; q2 < 32; ++q2) {
      const int r = 64 * wave + 2 * q2 + hl;
      const uint4 v = *reinterpret_cast<const uint4*>(ring + r * 512 + ((chunk ^ (r & 15)) << 4));
      const int mrow = m0 + r;
      if (mrow >= g.m || col >= g.n) continue;
      if (EPI == EPI_RESIDUAL || (EPI == EPI_STREAM && g.r != nullptr)) {
        const uint4 rv = *reinterpret_cast<const uint4*>(g.r + mrow * g.ldr + col);
        *reinterpret_cast<uint4*>(g.c + mrow * g.ldc + col) = make_uint4(
            add_bf16x2(rv.x, v.x), add_bf16x2(rv.y, v.y), add_bf16x2(rv.z, v.z), add_bf16x2(rv.w, v.w));
      } else {
        *reinterpret_cast<uint4*>(g.c + mrow * g.ldc + col) = v;
      }
    }
    if constexpr (EPI == EPI_STREAM) {
      wait_lds();
      bar();
    }
  }
}

// Lane offsets (bytes) of the 8 runs of wave q's quarter of an operand's
// stage in a whole tile (no clamping), relative to the wave's base: the
// operand at row (KC) or column (KO) o0 + 64q, k 0.  The same as RunPlan's
// (KC: row 8jj + lane/8, the chunk the swizzle puts in slot lane%8; KO: k row
// 8jj + (lane%16)/2, chunk 2 (lane/16) + lane%2), so the tiles agree.  Leading
// dims below 2^24 keep them in range.
template <bool KO>
__device__ __forceinline__ void whole_run_offsets(int64_t ld, int lane, uint32_t (&off)[8]) {
  const uint32_t l = static_cast<uint32_t>(ld);
  if constexpr (KO) {
    const int r = (lane >> 1) & 7, c = 2 * (lane >> 4) + (lane & 1);
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) off[jj] = (static_cast<uint32_t>(8 * jj + r) * l + 8u * c) * 2u;
  } else {
    const int lr = lane >> 3;
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      const int c = (lane & 7) ^ swz<64>(8 * jj + lr);
      off[jj] = (static_cast<uint32_t>(8 * jj + lr) * l + 8u * c) * 2u;
    }
  }
}

// Wave q's base (bytes) of an operand in the tile at o0 (rows for KC,
// columns for KO).
template <bool KO>
__device__ __forceinline__ const char* whole_base(const uint16_t* base, int64_t ld, int o0, int q) {
  return reinterpret_cast<const char*>(base + (KO ? static_cast<int64_t>(o0 + 64 * q)
                                                   : static_cast<int64_t>(o0 + 64 * q) * ld));
}

// Persistent whole-K form with plain stores (no residual, no rotation; K of
// at least two stages; m and n multiples of the tile; more tiles than
// workgroups): one workgroup per CU runs tiles lid, lid + G, lid + 2G, ... of
// the G workgroups (in k_gemm's XCD order).  The ring runs on across tiles:
// the loads issued in a tile's last two stages bring the next tile's first two,
// and
// the output goes from the accumulators straight to global memory (8
// consecutive columns per lane and store, gathered by a lane swap), with no
// LDS staging.  So the next tile's operands land while the epilogue runs, and
// its first stage needs no prologue.  Against one workgroup per tile
// this saves, per tile, the prologue (two stages loaded and the first waited
// for), the output's round trip through LDS with its barriers, and the gap
// between a CU's consecutive workgroups.
template <bool A_KO, bool B_KO, bool RESID>
__device__ __forceinline__ void gemm_persist(const GemmArgs& g, char* ring, int lid) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  const int nst = g.total_steps;
  int t = lid, m0, n0;
  tile_origin(g, t, m0, n0);
  uint32_t offa[8], offb[8];
  whole_run_offsets<A_KO>(g.lda, lane, offa);
  whole_run_offsets<B_KO>(g.ldb, lane, offb);
  const int64_t kba = A_KO ? g.lda * 2 : 2, kbb = B_KO ? g.ldb * 2 : 2;  // bytes per k
  const char* ba = whole_base<A_KO>(g.a, g.lda, m0, wave);
  const char* bb = whole_base<B_KO>(g.b, g.ldb, n0, wave);
  typedef __attribute__((address_space(3))) char* lptr;
  const uint32_t ring0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lptr)ring)) + wave * 8192;

  const int wm16 = 128 * wm, wn16 = 128 * wn;
  const int a_off = lane_off_kc16(lane);
  const int t0 = lane_off_tr16(lane);
  bf16x8 fa[2][8], fb[2][8];
  auto rd1 = [&](int sa, int sb, int ks, int buf, int r) __attribute__((always_inline)) {
    if (r >= 1 && r <= 8) {
      const char* tile = ring + sa * kSlot;
      const int j = r - 1, o = wm16 + 16 * j;
      fa[buf][j] = A_KO ? frag_ko16(tile, t0, o, ks) : frag_kc16(tile, a_off, o, ks);
    } else {
      const char* tile = ring + sb * kSlot;
      const int i = r == 0 ? 0 : r - 8, o = wn16 + 16 * i;
      fb[buf][i] = B_KO ? frag_ko16(tile, t0, o, ks) : frag_kc16(tile, a_off, o, ks);
    }
  };
  f32x4 acc[8][8];
  auto mf1 = [&](int buf, int nn) __attribute__((always_inline)) {
    const int i = nn >> 3, j = nn & 7;
    acc[i][j] = mfma16(fb[buf][i], fa[buf][j], acc[i][j]);
  };

  // Prologue of the first tile (as gemm_tile's).
#pragma unroll
  for (int jj = 0; jj < 8; ++jj) dma16(offa[jj], ba, ring0 + 0 * kSlot + jj * 1024);
#pragma unroll
  for (int jj = 0; jj < 8; ++jj) dma16(offb[jj], bb, ring0 + 1 * kSlot + jj * 1024);
#pragma unroll
  for (int jj = 0; jj < 8; ++jj) dma16(offa[jj], ba + kTk * kba, ring0 + 2 * kSlot + jj * 1024);
#pragma unroll
  for (int jj = 0; jj < 8; ++jj) dma16(offb[jj], bb + kTk * kbb, ring0 + 3 * kSlot + jj * 1024);
  wait_vm_n<16>();
  bar();
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    rd1(0, 1, 0, 0, r);
    __builtin_amdgcn_sched_barrier(0);
  }

  int s = 0;  // ring slot of the current stage's A (stage x: A in s, B in s+1)
  for (;;) {
    const int tn = t + g.grid;
    const bool more = tn < g.tiles;
    int m1 = m0, n1 = n0;
    if (more) tile_origin(g, tn, m1, n1);
    const char* na = whole_base<A_KO>(g.a, g.lda, m1, wave);
    const char* nb = whole_base<B_KO>(g.b, g.ldb, n1, wave);
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    // Stage x (as gemm_tile's): the loads issued in it are stage x + 2's, of
    // this tile, of the next, or past the last tile's end (its last stage
    // again: in bounds, never used).
    for (int x = 0; x < nst; ++x) {
      const int sB = mod5(s + 1), nA = mod5(s + 2), nB = mod5(s + 3), fA = mod5(s + 4);
      const bool ahead = more && x + 2 >= nst;
      const int64_t k2 = static_cast<int64_t>(ahead ? x + 2 - nst : min(x + 2, nst - 1)) * kTk;
      const char* srcA = (ahead ? na : ba) + k2 * kba;
      const char* srcB = (ahead ? nb : bb) + k2 * kbb;
      const uint32_t dA = ring0 + fA * kSlot, dB = ring0 + s * kSlot;
      asm volatile("s_nop 4");
#pragma unroll
      for (int p = 0; p < 64; ++p) {
        if ((p & 3) == 0) rd1(s, sB, 1, 1, p >> 2);
        if ((p & 7) == 1) set_m0(dA + (p >> 3) * 1024);
        if ((p & 7) == 2) dma16_m0(offa[p >> 3], srcA);
        mf1(0, p);
        __builtin_amdgcn_sched_barrier(0);
      }
      wait_lds();
      wait_vm_n<8>();
      bar();
#pragma unroll
      for (int p = 0; p < 64; ++p) {
        if ((p & 3) == 0) rd1(nA, nB, 0, 0, p >> 2);
        if ((p & 7) == 1) set_m0(dB + (p >> 3) * 1024);
        if ((p & 7) == 2) dma16_m0(offb[p >> 3], srcB);
        mf1(1, p);
        __builtin_amdgcn_sched_barrier(0);
      }
      s = nA;
      // MFMA results need wait states before the epilogue reads them.
      if (x == nst - 1) asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7");
    }
    __builtin_amdgcn_sched_barrier(0);
    // Lane i of accumulator (i, j) holds row 128 wm + 16 j + i%16, columns
    // 128 wn + 16 i + 4 g .. +3 (g = i/16, its row of 16 lanes).  For a pair
    // of accumulators (i, i+1), one v_permlane16_swap per dword trades the
    // odd rows' block-i columns for the even rows' block-(i+1) columns, after
    // which lane g holds 8 consecutive columns, 8 (g/2) .. +7 of block
    // i + g%2: one 16-byte store (64 contiguous bytes per row and store).
    // The form runs whole tiles only.
    const int64_t lane_row = m0 + wm16 + (lane & 15);
    const int lane_col = n0 + wn16 + 16 * ((lane >> 4) & 1) + 8 * (lane >> 5);
    uint16_t* cp = g.c + lane_row * g.ldc + lane_col;
    // RESID: C = bf16(R + bf16(A B^T)) (R may be C itself: each lane reads its
    // own chunks before it writes them).  All 32 residual chunks are loaded
    // before the first store, so no load waits behind a store that might
    // alias it.
    uint4 rv[RESID ? 32 : 1];
    if constexpr (RESID) {
      const uint16_t* rp = g.r + lane_row * g.ldr + lane_col;
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          rv[4 * j + q] = *reinterpret_cast<const uint4*>(rp + static_cast<int64_t>(16 * j) * g.ldr + 32 * q);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x4 v0 = acc[2 * q][j], v1 = acc[2 * q + 1][j];
        const auto lo = __builtin_amdgcn_permlane16_swap(pk_bf16(v0[0], v0[1]), pk_bf16(v1[0], v1[1]), false, false);
        const auto hi = __builtin_amdgcn_permlane16_swap(pk_bf16(v0[2], v0[3]), pk_bf16(v1[2], v1[3]), false, false);
        uint4 o = make_uint4(lo[0], hi[0], lo[1], hi[1]);
        if constexpr (RESID) {
          const uint4 r = rv[4 * j + q];
          o = make_uint4(add_bf16x2(r.x, o.x), add_bf16x2(r.y, o.y), add_bf16x2(r.z, o.z), add_bf16x2(r.w, o.w));
        }
        *reinterpret_cast<uint4*>(cp + static_cast<int64_t>(16 * j) * g.ldc + 32 * q) = o;
      }
    __builtin_amdgcn_sched_barrier(0);
    if (!more) break;
    t = tn;
    m0 = m1;
    n0 = n1;
    ba = na;
    bb = nb;
  }
  // The loads past the last tile's end land before the workgroup's LDS is
  // released.
  wait_vm();
  wait_lds();
}

// One tile, or one K slice of a tile (EPI_PARTIAL), per workgroup; or the
// stream form (EPI_STREAM): the workgroup runs its whole tiles, then its share
// of the tail's k-steps as segments of one tile each.  A tail segment that is not a whole tile goes to
// fp32 slot 2w (the workgroup's first tail segment) or 2w + 1 (its last);
// k_gemm_fixup adds a split tile's segments in k order.
template <bool A_KO, bool B_KO, int EPI>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void k_gemm(GemmArgs g) {
  __shared__ __align__(16) char ring[kRing * kSlot];
  const int nb8 = gridDim.x >> 3;
  const int lid = (blockIdx.x & 7) * nb8 + (blockIdx.x >> 3);
  if (lid >= g.grid) return;
  if constexpr (EPI == EPI_STREAM) {
    // One call site for both kinds of segment (one copy of the main loop).
    // Tail: linear, workgroup lid takes tail k-steps [lid I / G, (lid + 1) I / G)
    // of the tail tiles in order; or in XCD slabs (slab_chunks > 0, the tail a
    // whole number C of chunks of P = G / 8 consecutive tiles): the P
    // workgroups of XCD x (lids x P .. x P + P - 1, blockIdx % 8 == x) take
    // chunk-k-steps [x W / 8, (x + 1) W / 8) of the W = C * ki, workgroup
    // x P + j tile j of each chunk, so an XCD's workgroups run one chunk's
    // tiles over the same k-steps together and share their operand blocks in
    // L2, as in the whole rounds.  A slab is shorter than ki (C < 8): every
    // tail tile is split.
    const int64_t ki = g.total_steps;
    const int P = g.grid >> 3, xcd = lid / P, j = lid - xcd * P;
    const int64_t W = static_cast<int64_t>(g.slab_chunks) * ki;
    const int64_t beg = g.slab_chunks ? xcd * W / 8 : lid * g.tail_iters / g.grid;
    const int64_t end = g.slab_chunks ? (xcd + 1) * W / 8 : (lid + 1) * g.tail_iters / g.grid;
    int r = 0;
    for (int64_t it = beg;;) {
      int t, k0 = 0, len = g.total_steps;
      float* slot = nullptr;
      if (r < g.full_rounds) {
        t = r++ * g.grid + lid;
      } else if (it < end) {
        const int q = static_cast<int>(it / ki);  // tail tile, or chunk
        k0 = static_cast<int>(it - q * ki);
        len = static_cast<int>(min(ki - k0, end - it));
        t = g.full_rounds * g.grid + (g.slab_chunks ? q * P + j : q);
        slot = g.part + (2 * static_cast<int64_t>(lid) + (it == beg ? 0 : 1)) * (kTm * kTn);
        it += len;
      } else {
        break;
      }
      const GemmArgs pg = for_tile(g, t);
      gemm_tile<A_KO, B_KO, EPI>(pg, ring, t, k0, len, slot, kTn, len < ki);
    }
  } else {
    const int slice = lid / g.tiles, t = lid - slice * g.tiles;
    const int s_begin = slice * g.steps_per_slice;
    int m0, n0;
    tile_origin(g, t, m0, n0);
    float* pdst = EPI == EPI_PARTIAL
                      ? g.part + static_cast<int64_t>(slice) * g.m * g.n + static_cast<int64_t>(m0) * g.n + n0
                      : nullptr;
    gemm_tile<A_KO, B_KO, EPI>(g, ring, t, s_begin, min(g.total_steps - s_begin, g.steps_per_slice), pdst,
                               g.n, EPI == EPI_PARTIAL);
  }
}

// The persistent form (gemm_persist): G = gridDim.x workgroups, a multiple of
// 8, at most the number of tiles.
template <bool A_KO, bool B_KO, bool RESID>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void k_gemm_persist(GemmArgs g) {
  __shared__ __align__(16) char ring[kRing * kSlot];
  const int nb8 = gridDim.x >> 3;
  gemm_persist<A_KO, B_KO, RESID>(g, ring, (blockIdx.x & 7) * nb8 + (blockIdx.x >> 3));
}

// Rows blockIdx.y * 16 .. +15 of tail tile blockIdx.x of a stream GEMM: if
// more than one workgroup's k-range meets the tile (always, with XCD slabs),
// C = bf16(sum of their fp32 segments in k order) (+ residual, rounded as
// k_gemm_reduce).  A holder's first segment is in its slot 0, a second in
// slot 1.  Thread (row group, lane) adds 4 columns of 4 rows, one contributor
// at a time (its 4 loads in flight together).
constexpr int kFixRows = 16;

__global__ __launch_bounds__(256) void k_gemm_fixup(GemmArgs g) {
  // Holders of the tile's k-steps: workgroups w (linear) or the XCDs w of the
  // tile's chunk c, whose workgroup w P + j holds tile j of it (slabs); in
  // both, holder w covers [w I / N, (w + 1) I / N) of I steps over N holders,
  // so the one holding step i is ceil((i + 1) N / I) - 1.
  const int64_t ki = g.total_steps, G = g.grid, P = G >> 3;
  const bool slab = g.slab_chunks > 0;
  const int64_t I = slab ? g.slab_chunks * ki : g.tail_iters, N = slab ? 8 : G;
  const int64_t c = slab ? blockIdx.x / P : blockIdx.x, jj = slab ? blockIdx.x - c * P : 0;
  const int64_t lo = c * ki;
  auto wg_of = [&](int64_t i) { return static_cast<int>(((i + 1) * N + I - 1) / I - 1); };
  auto start_of = [&](int64_t w) { return w * I / N; };
  const int w0 = wg_of(lo), w1 = wg_of(lo + ki - 1);
  if (w0 == w1 && !slab) return;  // one workgroup stored the whole tile
  int m0, n0, tl = g.full_rounds * g.grid + static_cast<int>(blockIdx.x);
  const GemmArgs pg = for_tile(g, tl);  // the tile's problem: pg.c, pg.r, pg.m, pg.n
  tile_origin(pg, tl, m0, n0);
  const int lane = threadIdx.x & 63, r0 = blockIdx.y * kFixRows + (threadIdx.x >> 6);
  const int col = n0 + 4 * lane;
  if (col >= pg.n) return;
  float4 acc[kFixRows / 4];
  bool first = true;
  for (int w = w0; w <= w1; ++w) {
    const int64_t sw = start_of(w);
    if (sw == start_of(w + 1)) continue;  // empty range: wrote nothing
    const int64_t holder = slab ? w * P + jj : w;
    const float* src = g.part + (2 * holder + (sw >= lo ? 0 : 1)) * (kTm * kTn) + 4 * lane;
    float4 v[kFixRows / 4];
#pragma unroll
    for (int q = 0; q < kFixRows / 4; ++q) v[q] = *reinterpret_cast<const float4*>(src + (r0 + 4 * q) * kTn);
#pragma unroll
    for (int q = 0; q < kFixRows / 4; ++q) {
      if (first) {
        acc[q] = v[q];
      } else {
        acc[q].x += v[q].x;
        acc[q].y += v[q].y;
        acc[q].z += v[q].z;
        acc[q].w += v[q].w;
      }
    }
    first = false;
  }
#pragma unroll
  for (int q = 0; q < kFixRows / 4; ++q) {
    const int mrow = m0 + r0 + 4 * q;
    if (mrow >= pg.m) break;
    float4 s = acc[q];
    if (pg.r != nullptr) {
      const uint2 rv = *reinterpret_cast<const uint2*>(pg.r + static_cast<int64_t>(mrow) * pg.ldr + col);
      s.x = __uint_as_float(rv.x << 16) + round_bf(s.x);
      s.y = __uint_as_float(rv.x & 0xffff0000u) + round_bf(s.y);
      s.z = __uint_as_float(rv.y << 16) + round_bf(s.z);
      s.w = __uint_as_float(rv.y & 0xffff0000u) + round_bf(s.w);
    }
    *reinterpret_cast<uint2*>(pg.c + static_cast<int64_t>(mrow) * pg.ldc + col) =
        make_uint2(pk_bf16(s.x, s.y), pk_bf16(s.z, s.w));
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

// Compute units of the current device (one workgroup fits per CU), looked up
// once per device (std::call_once, so concurrent first calls are safe).
int device_cus() {
  constexpr int kMaxDevices = 64;
  static std::once_flag once[kMaxDevices];
  static int cached[kMaxDevices] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
  std::call_once(once[dev], [dev]() {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      cus = 256;
    cached[dev] = cus;
  });
  return cached[dev];
}

// Workgroups of a stream GEMM: one per CU, a multiple of 8 (the XCD order).
int stream_grid() { return std::max(8, device_cus() / 8 * 8); }

// How a GEMM is split.  Modelled times, in rounds of a whole-K tile:
//   K slices S: ceil(tiles*S / CUs) / S, plus for S > 1 writing and re-reading
//     the S fp32 partial outputs (8 bytes per output and slice at ~5 TB/s,
//     against a whole-K tile's MFMA time at ~6 TFLOP/s per CU); every slice
//     keeps at least 256 k.
//   stream: floor(tiles / CUs) whole rounds, then the remaining tiles' k-steps
//     split evenly over the CUs (tail_tiles / CUs), plus the fp32 traffic of
//     the split tiles' segments (at most CUs + tail_tiles of them, 256 x 256
//     each).  Plain stores and the residual epilogue (not the rotation).
//     Only with at least one whole round: with fewer tiles than CUs every
//     workgroup starts at another k offset, so the workgroups of an XCD no
//     longer share operand blocks in L2 (TN 2048 x 5632 x 16384, 176 tiles:
//     450 us against 361 us split in 4; 11264 x 2048, 352 tiles: 655-660
//     against 685 us, 10240 x 2048: 644-666 against 754 us).
struct GemmPlan {
  int slices;   // K slices of the split form
  bool stream;  // the stream form models faster
};

GemmPlan gemm_plan(int64_t m, int64_t n, int64_t k) {
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
  GemmPlan p{static_cast<int>((steps + per - 1) / per), false};
  const int64_t sg = stream_grid(), tail = tiles % sg;
  if (tiles > sg && tail > 0 && steps >= 4) {
    const double segs = static_cast<double>(std::min<int64_t>(2 * sg, sg + tail));
    const double cost = static_cast<double>(tiles / sg) + static_cast<double>(tail) / sg +
                        per_slice * segs * (kTm * kTn) / (static_cast<double>(m) * n);
    p.stream = cost < 0.97 * best_cost;
  }
  return p;
}

size_t stream_workspace_bytes() { return 2 * static_cast<size_t>(stream_grid()) * kTm * kTn * sizeof(float); }

template <bool A_KO, bool B_KO>
void launch(const GemmArgs& g, unsigned blocks, bool partial, bool resid, hipStream_t stream) {
  if constexpr (!A_KO && !B_KO) {  // the rotated forward projection is NT only
    if (g.rope.cos) {
      hipLaunchKernelGGL((k_gemm<false, false, EPI_ROPE>), dim3(blocks), dim3(256), 0, stream, g);
      return;
    }
  }
  if (g.tail_iters > 0)
    hipLaunchKernelGGL((k_gemm<A_KO, B_KO, EPI_STREAM>), dim3(blocks), dim3(256), 0, stream, g);
  else if (partial)
    hipLaunchKernelGGL((k_gemm<A_KO, B_KO, EPI_PARTIAL>), dim3(blocks), dim3(256), 0, stream, g);
  else if (resid)
    hipLaunchKernelGGL((k_gemm<A_KO, B_KO, EPI_RESIDUAL>), dim3(blocks), dim3(256), 0, stream, g);
  else
    hipLaunchKernelGGL((k_gemm<A_KO, B_KO, EPI_STORE>), dim3(blocks), dim3(256), 0, stream, g);
}

bool valid_op(int op) { return op == FH_GEMM_NT || op == FH_GEMM_NN || op == FH_GEMM_TN; }

}  // namespace
}  // namespace fh

using namespace fh;

extern "C" size_t fh_gemm_bf16_workspace_size(int op, int64_t m, int64_t n, int64_t k) {
  if (!valid_op(op) || m <= 0 || n <= 0 || k <= 0 || k % 64) return 0;
  // the stream form's segment slots, or the split form's partials
  const GemmPlan p = gemm_plan(m, n, k);
  if (p.stream) return stream_workspace_bytes();
  return p.slices > 1 ? static_cast<size_t>(p.slices) * m * n * sizeof(float) : 0;
}

namespace {

// Checks the operands of one GEMM and fills g (tiling for `slices` K slices).
int gemm_setup(int op, const void* a, int64_t lda, const void* b, int64_t ldb, void* c, int64_t ldc,
               const void* residual, int64_t ldr, int64_t m, int64_t n, int64_t k, GemmArgs& g) {
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
  FH_REQUIRE(lda >= a_cols && ldb >= b_cols && ldc >= n && lda % 8 == 0 && ldb % 8 == 0 && ldc % 8 == 0,
             "gemm_bf16: leading dims must cover the rows and be multiples of 8");
  FH_REQUIRE(a && b && c, "gemm_bf16: null pointer");
  FH_REQUIRE(aligned16(a) && aligned16(b) && aligned16(c), "gemm_bf16: a, b and c must be 16-byte aligned");
  if (residual) {
    FH_REQUIRE(ldr >= n && ldr % 8 == 0 && aligned16(residual),
               "gemm_bf16: residual must be 16-byte aligned with ldr >= n, a multiple of 8");
    FH_REQUIRE(residual == c ? ldr == ldc : true, "gemm_bf16: residual aliasing c must share its ldc");
  }
  g = GemmArgs{};
  g.a = static_cast<const uint16_t*>(a);
  g.b = static_cast<const uint16_t*>(b);
  g.c = static_cast<uint16_t*>(c);
  g.r = static_cast<const uint16_t*>(residual);
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
  g.ngroup = 1;
  g.grp[0] = GemmProblem{g.a, g.b, g.c, g.r, lda, ldb, ldc, ldr, g.m, g.n, g.tiles_m, g.tiles_n, 0};
  return FH_OK;
}

// Launches the GEMM of g in the stream form (stream: segment slots in
// `workspace`, split tiles summed by k_gemm_fixup) or over `slices` K slices
// (partials in `workspace`, summed by k_gemm_reduce, when slices > 1).
int gemm_run(int op, GemmArgs& g, int slices, bool stream_form, void* workspace, hipStream_t stream) {
  g.part = static_cast<float*>(workspace);
  if (stream_form) {
    const int sg = stream_grid();
    g.grid = sg;
    g.full_rounds = g.tiles / sg;
    g.tail_tiles = g.tiles - g.full_rounds * sg;
    g.tail_iters = static_cast<int64_t>(g.tail_tiles) * g.total_steps;
    g.steps_per_slice = g.total_steps;
    g.slab_chunks = g.tail_tiles % (sg / 8) == 0 ? g.tail_tiles / (sg / 8) : 0;
    switch (op) {
      case FH_GEMM_NT: launch<false, false>(g, sg, false, false, stream); break;
      case FH_GEMM_NN: launch<false, true>(g, sg, false, false, stream); break;
      default: launch<true, true>(g, sg, false, false, stream); break;
    }
    if (g.tail_tiles > 0)
      hipLaunchKernelGGL(k_gemm_fixup, dim3(g.tail_tiles, kTm / kFixRows), dim3(256), 0, stream, g);
    return FH_OK;
  }
  g.steps_per_slice = (g.total_steps + slices - 1) / slices;
#if FH_GEMM_PERSIST
  // The residual epilogue in this form: the forward (NT) layout only.
  if (slices == 1 && (g.r == nullptr || op == FH_GEMM_NT) && g.rope.cos == nullptr && g.total_steps >= 2 &&
      g.m % kTm == 0 && g.n % kTn == 0 && g.lda < (int64_t(1) << 24) && g.ldb < (int64_t(1) << 24) &&
      g.tiles > stream_grid()) {
    g.grid = stream_grid();
    if (g.r != nullptr) {
      hipLaunchKernelGGL((k_gemm_persist<false, false, true>), dim3(g.grid), dim3(256), 0, stream, g);
      return FH_OK;
    }
    switch (op) {
      case FH_GEMM_NT: hipLaunchKernelGGL((k_gemm_persist<false, false, false>), dim3(g.grid), dim3(256), 0, stream, g); break;
      case FH_GEMM_NN: hipLaunchKernelGGL((k_gemm_persist<false, true, false>), dim3(g.grid), dim3(256), 0, stream, g); break;
      default: hipLaunchKernelGGL((k_gemm_persist<true, true, false>), dim3(g.grid), dim3(256), 0, stream, g); break;
    }
    return FH_OK;
  }
#endif
  const int64_t logical = static_cast<int64_t>(g.tiles) * slices;
  FH_REQUIRE(logical <= 0x7ffffff0, "gemm_bf16: grid too large");
  g.grid = static_cast<int>(logical);
  const unsigned blocks = static_cast<unsigned>((logical + 7) / 8 * 8);
  const bool partial = slices > 1, resid = g.r != nullptr;
  switch (op) {
    case FH_GEMM_NT: launch<false, false>(g, blocks, partial, resid, stream); break;
    case FH_GEMM_NN: launch<false, true>(g, blocks, partial, resid, stream); break;
    default: launch<true, true>(g, blocks, partial, resid, stream); break;
  }
  if (partial) {
    const int64_t mn = static_cast<int64_t>(g.m) * g.n;
    const unsigned rb = static_cast<unsigned>((mn / 4 + 255) / 256);
    if (resid)
      hipLaunchKernelGGL(k_gemm_reduce<true>, dim3(rb), dim3(256), 0, stream, g.part, slices, g.m, g.n, g.c,
                         g.ldc, g.r, g.ldr);
    else
      hipLaunchKernelGGL(k_gemm_reduce<false>, dim3(rb), dim3(256), 0, stream, g.part, slices, g.m, g.n,
                         g.c, g.ldc, nullptr, int64_t(0));
  }
  return FH_OK;
}

}  // namespace

extern "C" int fh_gemm_bf16(int op, const void* a, int64_t lda, const void* b, int64_t ldb, void* c,
                            int64_t ldc, const void* residual, int64_t ldr, int64_t m, int64_t n,
                            int64_t k, void* workspace, hipStream_t stream) {
  GemmArgs g;
  if (int e = gemm_setup(op, a, lda, b, ldb, c, ldc, residual, ldr, m, n, k, g)) return e;
  const GemmPlan p = gemm_plan(m, n, k);
  FH_REQUIRE((p.slices == 1 && !p.stream) || (workspace && aligned16(workspace)),
             "gemm_bf16: workspace (fh_gemm_bf16_workspace_size bytes) required");
  if (int e = gemm_run(op, g, p.slices, p.stream, workspace, stream)) return e;
  return check_launch("fh_gemm_bf16");
}

namespace {

// A group runs as one stream launch when its tiles fill more than a round of
// the CUs (the tail, if any, in XCD slabs when it is a whole number of
// 32-tile chunks); otherwise its problems run one by one, each by its own plan.
bool group_stream(int64_t tiles, int64_t steps) { return tiles > stream_grid() && steps >= 4; }

// Checks every problem of a group and fills g with the group's table (tiles
// numbered problem by problem).
int group_setup(int op, int count, const fh_gemm_problem* probs, int64_t k, GemmArgs& g) {
  FH_REQUIRE(count >= 1 && count <= kMaxGroup && probs != nullptr,
             "gemm_bf16_grouped: between 1 and 3 problems required");
  int tile0 = 0;
  for (int i = 0; i < count; ++i) {
    const fh_gemm_problem& p = probs[i];
    GemmArgs gi;
    if (int e = gemm_setup(op, p.a, p.lda, p.b, p.ldb, p.c, p.ldc, p.residual, p.ldr, p.m, p.n, k, gi)) return e;
    if (i == 0) g = gi;
    g.grp[i] = gi.grp[0];
    g.grp[i].tile0 = tile0;
    tile0 += gi.tiles;
  }
  g.ngroup = count;
  g.tiles = tile0;
  return FH_OK;
}

}  // namespace

extern "C" size_t fh_gemm_bf16_grouped_workspace_size(int op, int count, const fh_gemm_problem* problems,
                                                      int64_t k) {
  if (!valid_op(op) || count < 1 || count > kMaxGroup || problems == nullptr || k <= 0 || k % kTk) return 0;
  int64_t tiles = 0;
  size_t most = 0;
  for (int i = 0; i < count; ++i) {
    const int64_t m = problems[i].m, n = problems[i].n;
    if (m <= 0 || n <= 0) return 0;
    tiles += ((m + kTm - 1) / kTm) * ((n + kTn - 1) / kTn);
    most = std::max(most, fh_gemm_bf16_workspace_size(op, m, n, k));
  }
  return group_stream(tiles, k / kTk) ? stream_workspace_bytes() : most;
}

extern "C" int fh_gemm_bf16_grouped(int op, int count, const fh_gemm_problem* problems, int64_t k,
                                    void* workspace, hipStream_t stream) {
  GemmArgs g;
  if (int e = group_setup(op, count, problems, k, g)) return e;
  if (!group_stream(g.tiles, g.total_steps)) {
    for (int i = 0; i < count; ++i) {
      const fh_gemm_problem& p = problems[i];
      if (int e = fh_gemm_bf16(op, p.a, p.lda, p.b, p.ldb, p.c, p.ldc, p.residual, p.ldr, p.m, p.n, k,
                               workspace, stream))
        return e;
    }
    return FH_OK;
  }
  FH_REQUIRE(workspace && aligned16(workspace),
             "gemm_bf16_grouped: workspace (fh_gemm_bf16_grouped_workspace_size bytes) required");
  const int sg = stream_grid();
  g.part = static_cast<float*>(workspace);
  g.grid = sg;
  g.full_rounds = g.tiles / sg;
  g.tail_tiles = g.tiles - g.full_rounds * sg;
  g.tail_iters = static_cast<int64_t>(g.tail_tiles) * g.total_steps;
  g.steps_per_slice = g.total_steps;
  g.slab_chunks = g.tail_tiles % (sg / 8) == 0 ? g.tail_tiles / (sg / 8) : 0;
  switch (op) {
    case FH_GEMM_NT: hipLaunchKernelGGL((k_gemm<false, false, EPI_STREAM>), dim3(sg), dim3(256), 0, stream, g); break;
    case FH_GEMM_NN: hipLaunchKernelGGL((k_gemm<false, true, EPI_STREAM>), dim3(sg), dim3(256), 0, stream, g); break;
    default: hipLaunchKernelGGL((k_gemm<true, true, EPI_STREAM>), dim3(sg), dim3(256), 0, stream, g); break;
  }
  if (g.tail_tiles > 0)
    hipLaunchKernelGGL(k_gemm_fixup, dim3(g.tail_tiles, kTm / kFixRows), dim3(256), 0, stream, g);
  return check_launch("fh_gemm_bf16_grouped");
}

extern "C" int fh_gemm_bf16_rope(const void* a, int64_t lda, const void* b, int64_t ldb, void* c, int64_t ldc,
                                 int64_t m, int64_t n, int64_t k, int64_t rot_cols, int64_t head_dim,
                                 int64_t seq_len, const void* cos, const void* sin, int cos_per_token,
                                 hipStream_t stream) {
  GemmArgs g;
  if (int e = gemm_setup(FH_GEMM_NT, a, lda, b, ldb, c, ldc, nullptr, 0, m, n, k, g)) return e;
  FH_REQUIRE(head_dim == 32 || head_dim == 64 || head_dim == 128, "gemm_bf16_rope: head_dim must be 32, 64 or 128");
  FH_REQUIRE(rot_cols > 0 && rot_cols <= n && rot_cols % head_dim == 0,
             "gemm_bf16_rope: rot_cols must be a positive multiple of head_dim, at most n");
  FH_REQUIRE(seq_len > 0 && seq_len < (int64_t(1) << 30), "gemm_bf16_rope: seq_len out of range");
  FH_REQUIRE(cos_per_token || m % seq_len == 0, "gemm_bf16_rope: m must be a multiple of seq_len");
  FH_REQUIRE(cos && sin && aligned16(cos) && aligned16(sin), "gemm_bf16_rope: cos/sin null or not 16-byte aligned");
  g.rope.cos = static_cast<const uint16_t*>(cos);
  g.rope.sin = static_cast<const uint16_t*>(sin);
  g.rope.rot_cols = static_cast<int>(rot_cols);
  g.rope.hd = static_cast<int>(head_dim);
  g.rope.per_token = cos_per_token ? 1 : 0;
  g.rope.seq_len = static_cast<int>(seq_len);
  g.rope.seq = FastDiv(static_cast<uint32_t>(seq_len));
  if (int e = gemm_run(FH_GEMM_NT, g, 1, false, nullptr, stream)) return e;  // whole K: the epilogue sees final sums
  return check_launch("fh_gemm_bf16_rope");
}
