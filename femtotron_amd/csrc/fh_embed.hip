// Token embedding forward (row gather) and a deterministic backward
// (scatter-add without floating-point atomics).
//
// Reference: the embedding of the first pipeline stage
// (femtotron/model/llama_partial_model.py:181-184) is an nn.Embedding, which
// femtotron's TP plan replaces by VocabParallelEmbedding
// (femtotron/parallel/tensor_parallel/embedding.py:57-79).  At one rank that
// module is: ids outside [0, V) are masked to row 0, looked up with
// F.embedding, and their output rows zeroed; the backward of F.embedding sums
// the output gradients of all tokens with the same id into that id's row
// (nothing for masked tokens, nothing for nn.Embedding's padding_idx).
//
// Forward: one wave per token row, 128-bit loads/stores.  Backward:
//   1. keys[t] = id (V for masked / padding tokens), vals[t] = t;
//   2. a stable LSD radix sort of (key, t), 8-bit digits, 1024-key tiles:
//      per-tile digit histograms, one exclusive scan over (digit, tile),
//      a scatter whose in-tile ranks come from wave ballots (peers with the
//      same digit) plus per-wave digit counts in LDS; stability keeps every
//      id's tokens in ascending token order;
//   3. per id, the [start, end) range of its tokens in the sorted order;
//   4. one wave per vocabulary row: the row's gradient is the fp32 sum of its
//      tokens' output-gradient rows in token order, rounded once; rows with no
//      token are written as zeros (no separate clear).
// Integer atomics appear only in LDS histograms, whose counts do not depend on
// order; no float is ever summed in a run-dependent order.
#include "fh_common.hpp"

namespace fh {
namespace {

constexpr int kEmbThreads = 256;
constexpr int kRowsPerBlock = kEmbThreads / kWave;  // one row per wave
constexpr int kTile = 1024;                         // keys per sort block
constexpr int kRounds = kTile / kEmbThreads;
constexpr int kBins = 256;                          // 8-bit digits

size_t align256(size_t b) { return (b + 255) & ~size_t(255); }

// ------------------------------------------------------------- forward
template <typename T>
__global__ __launch_bounds__(kEmbThreads) void k_embed_fwd(const T* __restrict__ w,
                                                           const int64_t* __restrict__ ids,
                                                           T* __restrict__ out, int64_t n_tokens,
                                                           int64_t vocab, int64_t hidden) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
  if (t >= n_tokens) return;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t id = ids[t];
  const bool ok = id >= 0 && id < vocab;
  T* dst = out + t * hidden;
  if (ok) {
    const T* src = w + id * hidden;
    for (int64_t c = lane * 8; c < hidden; c += kWave * 8)
      Elem<T>::straw(dst + c, Elem<T>::ldraw(src + c));
  } else {
    const float z[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int64_t c = lane * 8; c < hidden; c += kWave * 8) Elem<T>::store8(dst + c, z);
  }
}

// ------------------------------------------------------------- backward
// Sort keys and values; clears the per-id ranges (threads i < vocab).
__global__ __launch_bounds__(kEmbThreads) void k_embed_keys(const int64_t* __restrict__ ids,
                                                            int64_t n_tokens, int64_t vocab,
                                                            int64_t padding_idx,
                                                            uint32_t* __restrict__ keys,
                                                            uint32_t* __restrict__ vals,
                                                            uint32_t* __restrict__ seg_start,
                                                            uint32_t* __restrict__ seg_end) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kEmbThreads + threadIdx.x;
  if (i < n_tokens) {
    const int64_t id = ids[i];
    const bool ok = id >= 0 && id < vocab && id != padding_idx;
    keys[i] = static_cast<uint32_t>(ok ? id : vocab);
    vals[i] = static_cast<uint32_t>(i);
  }
  if (i < vocab) {
    seg_start[i] = 0;
    seg_end[i] = 0;
  }
}

// Per-tile digit histogram, stored digit-major: hist[d * n_tiles + tile].
__global__ __launch_bounds__(kEmbThreads) void k_radix_hist(const uint32_t* __restrict__ keys,
                                                            int64_t n, int shift,
                                                            uint32_t* __restrict__ hist,
                                                            int n_tiles) {
  __shared__ uint32_t cnt[kBins];
  cnt[threadIdx.x] = 0;
  __syncthreads();
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kTile;
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    const int64_t i = base + r * kEmbThreads + threadIdx.x;
    if (i < n) atomicAdd(&cnt[(keys[i] >> shift) & (kBins - 1)], 1u);
  }
  __syncthreads();
  hist[static_cast<int64_t>(threadIdx.x) * n_tiles + blockIdx.x] = cnt[threadIdx.x];
}

// Exclusive scan of hist[0, m) in place by one block of 1024 threads: each
// thread owns one contiguous span; span totals are scanned in LDS.
__global__ __launch_bounds__(1024) void k_radix_scan(uint32_t* __restrict__ hist, int64_t m) {
  __shared__ uint32_t part[1024];
  const int64_t span = (m + 1023) / 1024;
  const int64_t lo = threadIdx.x * span;
  const int64_t hi = lo + span < m ? lo + span : m;
  uint32_t s = 0;
  for (int64_t i = lo; i < hi; ++i) s += hist[i];
  part[threadIdx.x] = s;
  __syncthreads();
  // Hillis-Steele inclusive scan of the 1024 span totals.
  for (int off = 1; off < 1024; off <<= 1) {
    const uint32_t add = threadIdx.x >= static_cast<unsigned>(off) ? part[threadIdx.x - off] : 0u;
    __syncthreads();
    part[threadIdx.x] += add;
    __syncthreads();
  }
  uint32_t run = threadIdx.x ? part[threadIdx.x - 1] : 0u;
  for (int64_t i = lo; i < hi; ++i) {
    const uint32_t c = hist[i];
    hist[i] = run;
    run += c;
  }
}

// Stable scatter of one tile.  Keys are taken in rounds of 256 (index order =
// (round, thread)); a key's position = scanned offset of (digit, tile) + keys
// of its digit in earlier rounds + in lower waves of this round + in lower
// lanes of its wave.
__global__ __launch_bounds__(kEmbThreads) void k_radix_scatter(
    const uint32_t* __restrict__ keys_in, const uint32_t* __restrict__ vals_in,
    uint32_t* __restrict__ keys_out, uint32_t* __restrict__ vals_out, int64_t n, int shift,
    const uint32_t* __restrict__ offsets, int n_tiles) {
  __shared__ uint32_t run[kBins];
  __shared__ uint32_t wcnt[kRowsPerBlock][kBins];
  const int lane = threadIdx.x & (kWave - 1);
  const int wv = threadIdx.x >> 6;
  const uint64_t lt_mask = (uint64_t(1) << lane) - 1;
  run[threadIdx.x] = 0;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kTile;
  for (int r = 0; r < kRounds; ++r) {
#pragma unroll
    for (int w = 0; w < kRowsPerBlock; ++w) wcnt[w][threadIdx.x] = 0;
    __syncthreads();
    const int64_t i = base + r * kEmbThreads + threadIdx.x;
    const bool valid = i < n;
    const uint32_t key = valid ? keys_in[i] : 0u;
    const uint32_t d = valid ? (key >> shift) & (kBins - 1) : kBins;  // kBins: no key
    uint64_t peers = ~uint64_t(0);
#pragma unroll
    for (int b = 0; b < 9; ++b) {
      const bool bit = (d >> b) & 1u;
      const uint64_t m = __ballot(bit);
      peers &= bit ? m : ~m;
    }
    const uint32_t rank = __popcll(peers & lt_mask);
    if (valid && rank == 0) wcnt[wv][d] = __popcll(peers);
    __syncthreads();
    if (valid) {
      uint32_t pos = run[d] + rank;
      for (int w = 0; w < wv; ++w) pos += wcnt[w][d];
      const uint64_t dst = static_cast<uint64_t>(offsets[static_cast<int64_t>(d) * n_tiles + blockIdx.x]) + pos;
      keys_out[dst] = key;
      vals_out[dst] = vals_in[i];
    }
    __syncthreads();
    uint32_t add = 0;
#pragma unroll
    for (int w = 0; w < kRowsPerBlock; ++w) add += wcnt[w][threadIdx.x];
    run[threadIdx.x] += add;
    // the next round's clear of wcnt is ordered after this read by its barrier
    __syncthreads();
  }
}

// [start, end) of every id's run in the sorted keys (sentinel key = vocab skipped).
__global__ __launch_bounds__(kEmbThreads) void k_embed_bounds(const uint32_t* __restrict__ keys,
                                                              int64_t n, uint32_t vocab,
                                                              uint32_t* __restrict__ seg_start,
                                                              uint32_t* __restrict__ seg_end) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kEmbThreads + threadIdx.x;
  if (i >= n) return;
  const uint32_t k = keys[i];
  if (k >= vocab) return;
  if (i == 0 || keys[i - 1] != k) seg_start[k] = static_cast<uint32_t>(i);
  if (i == n - 1 || keys[i + 1] != k) seg_end[k] = static_cast<uint32_t>(i + 1);
}

// One wave per vocabulary row: fp32 sum of the row's token gradients in token
// order.  Columns go in groups of kRowChunks x 512 (8 per lane per chunk) so
// that one token's loads for the whole group are in flight together.
constexpr int kRowChunks = 4;

template <typename T>
__global__ __launch_bounds__(kEmbThreads) void k_embed_rows(const T* __restrict__ dy,
                                                            const uint32_t* __restrict__ tok,
                                                            const uint32_t* __restrict__ seg_start,
                                                            const uint32_t* __restrict__ seg_end,
                                                            T* __restrict__ dw, int64_t vocab,
                                                            int64_t hidden) {
  const int64_t v = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
  if (v >= vocab) return;
  const int lane = threadIdx.x & (kWave - 1);
  const uint32_t lo = seg_start[v], hi = seg_end[v];
  T* dst = dw + v * hidden;
  for (int64_t c0 = lane * 8; c0 < hidden; c0 += kRowChunks * kWave * 8) {
    float acc[kRowChunks][8];
#pragma unroll
    for (int k = 0; k < kRowChunks; ++k)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[k][e] = 0.f;
    for (uint32_t j = lo; j < hi; ++j) {
      const T* src = dy + static_cast<int64_t>(tok[j]) * hidden + c0;
      float g[kRowChunks][8];
#pragma unroll
      for (int k = 0; k < kRowChunks; ++k)
        if (c0 + k * kWave * 8 < hidden) Elem<T>::load8(src + k * kWave * 8, g[k]);
#pragma unroll
      for (int k = 0; k < kRowChunks; ++k)
        if (c0 + k * kWave * 8 < hidden)
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[k][e] += g[k][e];
    }
#pragma unroll
    for (int k = 0; k < kRowChunks; ++k)
      if (c0 + k * kWave * 8 < hidden) Elem<T>::store8(dst + c0 + k * kWave * 8, acc[k]);
  }
}

int radix_passes(int64_t vocab) {
  int bits = 0;
  while ((int64_t(1) << bits) <= vocab) ++bits;  // keys take values 0..vocab
  return (bits + 7) / 8;
}

struct BwdLayout {
  size_t keys_a, vals_a, keys_b, vals_b, hist, seg_start, seg_end, total;
};

BwdLayout bwd_layout(int64_t n_tokens, int64_t vocab) {
  const int64_t tiles = (n_tokens + kTile - 1) / kTile;
  BwdLayout l{};
  size_t off = 0;
  const size_t keyb = align256(static_cast<size_t>(n_tokens) * 4);
  l.keys_a = off; off += keyb;
  l.vals_a = off; off += keyb;
  l.keys_b = off; off += keyb;
  l.vals_b = off; off += keyb;
  l.hist = off; off += align256(static_cast<size_t>(tiles) * kBins * 4);
  l.seg_start = off; off += align256(static_cast<size_t>(vocab) * 4);
  l.seg_end = off; off += align256(static_cast<size_t>(vocab) * 4);
  l.total = off;
  return l;
}

}  // namespace
}  // namespace fh

using namespace fh;

extern "C" int fh_embedding_fwd(fh_dtype dt, const void* weight, const int64_t* ids, void* out,
                                int64_t n_tokens, int64_t vocab, int64_t hidden,
                                hipStream_t stream) {
  FH_REQUIRE(dt == FH_BF16 || dt == FH_F32, "embedding_fwd: dtype must be FH_BF16 or FH_F32");
  FH_REQUIRE(n_tokens >= 0 && vocab > 0 && hidden > 0, "embedding_fwd: bad sizes");
  FH_REQUIRE(hidden % 8 == 0, "embedding_fwd: hidden must be a multiple of 8");
  if (n_tokens == 0) return FH_OK;
  FH_REQUIRE(weight && ids && out, "embedding_fwd: null pointer");
  FH_REQUIRE(aligned16(weight) && aligned16(out), "embedding_fwd: weight/out must be 16-byte aligned");
  FH_REQUIRE((n_tokens + kRowsPerBlock - 1) / kRowsPerBlock <= 0x7fffffff, "embedding_fwd: too many tokens");
  const dim3 grid(static_cast<unsigned>((n_tokens + kRowsPerBlock - 1) / kRowsPerBlock));
  if (dt == FH_BF16)
    hipLaunchKernelGGL(k_embed_fwd<uint16_t>, grid, dim3(kEmbThreads), 0, stream,
                       static_cast<const uint16_t*>(weight), ids, static_cast<uint16_t*>(out),
                       n_tokens, vocab, hidden);
  else
    hipLaunchKernelGGL(k_embed_fwd<float>, grid, dim3(kEmbThreads), 0, stream,
                       static_cast<const float*>(weight), ids, static_cast<float*>(out), n_tokens,
                       vocab, hidden);
  return check_launch("fh_embedding_fwd");
}

extern "C" size_t fh_embedding_bwd_workspace_size(int64_t n_tokens, int64_t vocab) {
  if (n_tokens < 0 || vocab <= 0) return 0;
  return bwd_layout(n_tokens, vocab).total;
}

extern "C" int fh_embedding_bwd(fh_dtype dt, const void* dy, const int64_t* ids, void* dweight,
                                int64_t n_tokens, int64_t vocab, int64_t hidden,
                                int64_t padding_idx, void* workspace, hipStream_t stream) {
  FH_REQUIRE(dt == FH_BF16 || dt == FH_F32, "embedding_bwd: dtype must be FH_BF16 or FH_F32");
  FH_REQUIRE(n_tokens >= 0 && vocab > 0 && hidden > 0, "embedding_bwd: bad sizes");
  FH_REQUIRE(hidden % 8 == 0, "embedding_bwd: hidden must be a multiple of 8");
  FH_REQUIRE(vocab < 0x7fffffff && n_tokens < 0x7fffffff, "embedding_bwd: sizes must fit 31 bits");
  FH_REQUIRE(dweight && workspace && (n_tokens == 0 || (dy && ids)), "embedding_bwd: null pointer");
  FH_REQUIRE(aligned16(dweight) && (n_tokens == 0 || aligned16(dy)) && aligned16(workspace),
             "embedding_bwd: dy/dweight/workspace must be 16-byte aligned");
  const BwdLayout l = bwd_layout(n_tokens, vocab);
  char* ws = static_cast<char*>(workspace);
  uint32_t* keys[2] = {reinterpret_cast<uint32_t*>(ws + l.keys_a), reinterpret_cast<uint32_t*>(ws + l.keys_b)};
  uint32_t* vals[2] = {reinterpret_cast<uint32_t*>(ws + l.vals_a), reinterpret_cast<uint32_t*>(ws + l.vals_b)};
  uint32_t* hist = reinterpret_cast<uint32_t*>(ws + l.hist);
  uint32_t* seg_start = reinterpret_cast<uint32_t*>(ws + l.seg_start);
  uint32_t* seg_end = reinterpret_cast<uint32_t*>(ws + l.seg_end);
  const int64_t wide = n_tokens > vocab ? n_tokens : vocab;
  hipLaunchKernelGGL(k_embed_keys, dim3(static_cast<unsigned>((wide + kEmbThreads - 1) / kEmbThreads)),
                     dim3(kEmbThreads), 0, stream, ids, n_tokens, vocab, padding_idx, keys[0], vals[0],
                     seg_start, seg_end);
  int cur = 0;
  if (n_tokens > 0) {
    const int tiles = static_cast<int>((n_tokens + kTile - 1) / kTile);
    const int passes = radix_passes(vocab);
    for (int p = 0; p < passes; ++p) {
      hipLaunchKernelGGL(k_radix_hist, dim3(tiles), dim3(kEmbThreads), 0, stream, keys[cur], n_tokens,
                         8 * p, hist, tiles);
      hipLaunchKernelGGL(k_radix_scan, dim3(1), dim3(1024), 0, stream, hist,
                         static_cast<int64_t>(tiles) * kBins);
      hipLaunchKernelGGL(k_radix_scatter, dim3(tiles), dim3(kEmbThreads), 0, stream, keys[cur],
                         vals[cur], keys[cur ^ 1], vals[cur ^ 1], n_tokens, 8 * p, hist, tiles);
      cur ^= 1;
    }
    hipLaunchKernelGGL(k_embed_bounds, dim3(static_cast<unsigned>((n_tokens + kEmbThreads - 1) / kEmbThreads)),
                       dim3(kEmbThreads), 0, stream, keys[cur], n_tokens, static_cast<uint32_t>(vocab),
                       seg_start, seg_end);
  }
  const dim3 grid(static_cast<unsigned>((vocab + kRowsPerBlock - 1) / kRowsPerBlock));
  if (dt == FH_BF16)
    hipLaunchKernelGGL(k_embed_rows<uint16_t>, grid, dim3(kEmbThreads), 0, stream,
                       static_cast<const uint16_t*>(dy), vals[cur], seg_start, seg_end,
                       static_cast<uint16_t*>(dweight), vocab, hidden);
  else
    hipLaunchKernelGGL(k_embed_rows<float>, grid, dim3(kEmbThreads), 0, stream,
                       static_cast<const float*>(dy), vals[cur], seg_start, seg_end,
                       static_cast<float*>(dweight), vocab, hidden);
  return check_launch("fh_embedding_bwd");
}
