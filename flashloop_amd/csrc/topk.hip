// J3: top-k selection by radix select.
//
//  * fl_decode_topk -- per (b,h) row of decode logits: the k highest-scoring keys
//    (ties -> lower index), ascending, zero padded to `capacity`, their softmax mass and
//    normalised weights (flashloop/engine.py:438-498, 84-109).
//  * fl_select_tokens -- per batch row of token scores: eligible candidates minus the
//    forced last token, top (count - forced), plus the last token
//    (flashloop/selection.py:26-69).
//
// One workgroup of 1024 threads per row.  Scores are mapped to order-preserving
// unsigned keys; four 8-bit histogram passes (LDS atomics) find the k-th largest key K*
// and how many keys equal to K* to take.  A final pass walks the row in index order,
// takes every key > K* and the first `need` keys == K* (ballot/popcount ranks), and
// writes the selected indices in ascending order.  The row stays in L2 across passes
// (131 KiB at 32K keys).
#include "fl_common.h"

namespace fl {
namespace {

constexpr int kTopkThreads = 1024;
constexpr int kTopkWaves = kTopkThreads / kWave;

__device__ __forceinline__ uint32_t order_key(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_value(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k ^ 0x80000000u) : ~k);
}

struct TopkShared {
  uint32_t hist[256];
  uint32_t wave_cnt[kTopkWaves];
  uint32_t wave_cnt2[kTopkWaves];
  float red[kTopkWaves];
  uint32_t sel_prefix;
  uint32_t sel_remaining;
  uint32_t bin_above;
};

__device__ float block_max(float v, TopkShared& sh) {
  v = wave_max(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh.red[w] = v;
  __syncthreads();
  float r = sh.red[0];
  for (int i = 1; i < kTopkWaves; ++i) r = fmaxf(r, sh.red[i]);
  return r;
}

__device__ float block_sum(float v, TopkShared& sh) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh.red[w] = v;
  __syncthreads();
  float r = 0.0f;
  for (int i = 0; i < kTopkWaves; ++i) r += sh.red[i];
  return r;
}

// Radix-select the k-th largest candidate key of the row.  On return (all threads):
// *kth = K*, *need = number of keys equal to K* to take (taking lowest indices first).
template <typename Cand>
__device__ void radix_select(const float* x, int n, int k, Cand cand, TopkShared& sh, uint32_t* kth, int* need) {
  uint32_t prefix = 0, mask = 0;
  int remaining = k;
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int i = threadIdx.x; i < 256; i += kTopkThreads) sh.hist[i] = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += kTopkThreads) {
      if (!cand(i)) continue;
      const uint32_t key = order_key(x[i]);
      if ((key & mask) == prefix) atomicAdd(&sh.hist[(key >> shift) & 0xFFu], 1u);
    }
    __syncthreads();
    if (threadIdx.x < kWave) {
      // lane l owns bins 255-4l .. 252-4l (descending); inclusive scan from the top
      const int l = threadIdx.x;
      uint32_t h[4];
      uint32_t local = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        h[e] = sh.hist[255 - 4 * l - e];
        local += h[e];
      }
      uint32_t incl = local;
#pragma unroll
      for (int off = 1; off < kWave; off <<= 1) {
        const uint32_t o = __shfl_up(incl, off, kWave);
        if (l >= off) incl += o;
      }
      uint32_t above = incl - local;  // keys in higher bins than this lane's
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (above < static_cast<uint32_t>(remaining) && above + h[e] >= static_cast<uint32_t>(remaining)) {
          sh.sel_prefix = 255 - 4 * l - e;
          sh.bin_above = above;
        }
        above += h[e];
      }
    }
    __syncthreads();
    prefix |= sh.sel_prefix << shift;
    mask |= 0xFFu << shift;
    remaining -= static_cast<int>(sh.bin_above);
    __syncthreads();
  }
  *kth = prefix;
  *need = remaining;
}

// Walk the row in index order; call emit(i, out_pos) for every selected candidate.
// Returns the number selected.
template <typename Cand, typename Emit>
__device__ int compact_selected(const float* x, int n, uint32_t kth, int need, Cand cand, TopkShared& sh, Emit emit) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  int eq_base = 0, out_base = 0;
  for (int base = 0; base < n; base += kTopkThreads) {
    const int i = base + threadIdx.x;
    bool gt = false, eq = false;
    if (i < n && cand(i)) {
      const uint32_t key = order_key(x[i]);
      gt = key > kth;
      eq = key == kth;
    }
    const uint64_t eq_ballot = __ballot(eq);
    if (lane == 0) sh.wave_cnt[w] = static_cast<uint32_t>(__popcll(eq_ballot));
    __syncthreads();
    int eq_rank = eq_base + __popcll(eq_ballot & lt_mask);
    int eq_total = 0;
    for (int j = 0; j < kTopkWaves; ++j) {
      const int c = static_cast<int>(sh.wave_cnt[j]);
      if (j < w) eq_rank += c;
      eq_total += c;
    }
    const bool sel = gt || (eq && eq_rank < need);
    const uint64_t sel_ballot = __ballot(sel);
    if (lane == 0) sh.wave_cnt2[w] = static_cast<uint32_t>(__popcll(sel_ballot));
    __syncthreads();
    int pos = out_base + __popcll(sel_ballot & lt_mask);
    int sel_total = 0;
    for (int j = 0; j < kTopkWaves; ++j) {
      const int c = static_cast<int>(sh.wave_cnt2[j]);
      if (j < w) pos += c;
      sel_total += c;
    }
    if (sel) emit(i, pos);
    eq_base += eq_total;
    out_base += sel_total;
    __syncthreads();
  }
  return out_base;
}

struct AllCand {
  __device__ bool operator()(int) const { return true; }
};

__global__ __launch_bounds__(kTopkThreads) void decode_topk_kernel(const float* scores, int64_t stride,
                                                                   const int32_t* n_keys, int rows_per_count,
                                                                   double fraction, int cap, int32_t* indices,
                                                                   uint8_t* valid, float* mass, float* weights,
                                                                   int32_t* counts) {
  __shared__ TopkShared sh;
  const int r = blockIdx.x;
  const float* x = scores + static_cast<int64_t>(r) * stride;
  const int n = min(n_keys[r / rows_per_count], static_cast<int>(min<int64_t>(stride, 0x7fffffff)));
  int32_t* oi = indices + static_cast<int64_t>(r) * cap;
  uint8_t* ov = valid + static_cast<int64_t>(r) * cap;
  float* ow = weights + static_cast<int64_t>(r) * cap;
  int k = 0;
  if (n > 0) {
    const double want = ceil(static_cast<double>(n) * fraction);
    k = static_cast<int>(want < 1.0 ? 1.0 : want);
    if (k > n) k = n;
  }
  if (k > cap) k = cap;  // caller-visible through counts
  if (k == 0) {
    for (int j = threadIdx.x; j < cap; j += kTopkThreads) {
      oi[j] = 0;
      ov[j] = 0;
      ow[j] = 0.0f;
    }
    if (threadIdx.x == 0) {
      mass[r] = 0.0f;
      if (counts) counts[r] = 0;
    }
    return;
  }
  // softmax statistics of the row (flashloop/engine.py:440-442)
  float mx = -INFINITY;
  for (int i = threadIdx.x; i < n; i += kTopkThreads) mx = fmaxf(mx, x[i]);
  const float M = block_max(mx, sh);
  float z = 0.0f;
  for (int i = threadIdx.x; i < n; i += kTopkThreads) z += fast_exp2((x[i] - M) * kLog2e);
  const float Z = block_sum(z, sh);
  const float invZ = 1.0f / Z;

  uint32_t kth;
  int need;
  radix_select(x, n, k, AllCand{}, sh, &kth, &need);
  float msum = 0.0f;
  compact_selected(x, n, kth, need, AllCand{}, sh, [&](int i, int pos) {
    const float w = fast_exp2((x[i] - M) * kLog2e) * invZ;
    oi[pos] = i;
    ov[pos] = 1;
    ow[pos] = w;
    msum += w;
  });
  const float S = block_sum(msum, sh);
  __threadfence_block();
  __syncthreads();
  const float invS = 1.0f / S;
  for (int j = threadIdx.x; j < cap; j += kTopkThreads) {
    if (j < k) {
      ow[j] = ow[j] * invS;
    } else {
      oi[j] = 0;
      ov[j] = 0;
      ow[j] = 0.0f;
    }
  }
  if (threadIdx.x == 0) {
    mass[r] = S;
    if (counts) counts[r] = k;
  }
}

// LDS-resident variant for rows of at most kLdsKeys keys (gfx950: 160 KiB of LDS per
// workgroup).  Passes over the row:
//   1. load from HBM into LDS as order-preserving keys (all loads issued first);
//   2. softmax normaliser and a histogram over kBins value-linear bins -- the bin is a
//      non-decreasing function of the score, so the k-th largest key lies in the bin B*
//      where the count from the top reaches k, and every key of a higher bin is larger;
//   3. the keys of B* (a few dozen for smooth score distributions) are compacted into an
//      LDS list and ranked there by (score desc, index asc), which fixes the k-th key
//      (kth_key, kth_idx) -- a bin too crowded for the list falls back to an exact radix
//      select restricted to B*;
//   4. the selected keys (key > kth_key, or key == kth_key and index <= kth_idx) are
//      written in index order: per (chunk, wave) ballot counts, one prefix scan, then
//      each lane writes at its offset.
constexpr int kLdsKeys = 35 * 1024;
constexpr int kPer = kLdsKeys / kTopkThreads;
constexpr int kSubHist = 4;
constexpr int kBins = kSubHist * 256;  // value-linear bins of the boundary search (one per thread)
constexpr int kCand = 512;             // boundary-bin list capacity
static_assert(kBins == kTopkThreads, "one boundary bin per thread");

// Non-decreasing in x; NaN products (inf - inf, 0 * inf) fall in bin 0, so the index is
// always in range.
__device__ __forceinline__ int value_bin(float x, float mn, float inv) {
  const float b = (x - mn) * inv;
  if (!(b > 0.0f)) return 0;
  return b >= static_cast<float>(kBins - 1) ? kBins - 1 : static_cast<int>(b);
}

struct LdsShared {
  uint32_t keys[kLdsKeys];
  uint32_t hist[kSubHist][256];
  uint32_t cnt[kPer][kTopkWaves];  // per (chunk, wave) counts, then their exclusive prefix
  uint32_t cand_key[kCand];
  uint32_t cand_idx[kCand];
  float red[kTopkWaves];
  uint32_t sel_digit;
  uint32_t bin_above;
  uint32_t ncand;
  uint32_t kth_key;
  uint32_t kth_idx;
};

__device__ float lds_block_max(float v, LdsShared& sh) {
  v = wave_max(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh.red[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = sh.red[0];
#pragma unroll
  for (int i = 1; i < kTopkWaves; ++i) r = fmaxf(r, sh.red[i]);
  return r;
}

__device__ float lds_block_sum(float v, LdsShared& sh) {
  v = wave_sum(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh.red[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = 0.0f;
#pragma unroll
  for (int i = 0; i < kTopkWaves; ++i) r += sh.red[i];
  return r;
}

// Exclusive prefix of sh.cnt in index order (chunk-major, wave-minor), done by wave 0;
// returns the total.  Caller brackets it with barriers.
__device__ uint32_t prefix_counts(LdsShared& sh) {
  __shared__ uint32_t total;
  if (threadIdx.x < kWave) {
    const int lane = threadIdx.x;
    constexpr int kN = kPer * kTopkWaves;
    constexpr int kEach = (kN + kWave - 1) / kWave;
    uint32_t* c = &sh.cnt[0][0];
    uint32_t loc[kEach];
    uint32_t sum = 0;
#pragma unroll
    for (int e = 0; e < kEach; ++e) {
      const int i = lane * kEach + e;
      loc[e] = i < kN ? c[i] : 0u;
      sum += loc[e];
    }
    uint32_t incl = sum;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const uint32_t o = __shfl_up(incl, off, kWave);
      if (lane >= off) incl += o;
    }
    uint32_t run = incl - sum;
#pragma unroll
    for (int e = 0; e < kEach; ++e) {
      const int i = lane * kEach + e;
      if (i < kN) c[i] = run;
      run += loc[e];
    }
    if (lane == kWave - 1) total = incl;
  }
  __syncthreads();
  return total;
}

__global__ __launch_bounds__(kTopkThreads) void decode_topk_lds_kernel(const float* scores, int64_t stride,
                                                                       const int32_t* n_keys, int rows_per_count,
                                                                       double fraction, int cap, int32_t* indices,
                                                                       uint8_t* valid, float* mass, float* weights,
                                                                       int32_t* counts) {
  __shared__ LdsShared sh;
  const int r = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const float* x = scores + static_cast<int64_t>(r) * stride;
  int n = min(n_keys[r / rows_per_count], static_cast<int>(min<int64_t>(stride, 0x7fffffff)));
  n = min(n, kLdsKeys);
  int32_t* oi = indices + static_cast<int64_t>(r) * cap;
  uint8_t* ov = valid + static_cast<int64_t>(r) * cap;
  float* ow = weights + static_cast<int64_t>(r) * cap;
  int k = 0;
  if (n > 0) {
    const double want = ceil(static_cast<double>(n) * fraction);
    k = static_cast<int>(want < 1.0 ? 1.0 : want);
    if (k > n) k = n;
  }
  if (k > cap) k = cap;
  for (int j = k + tid; j < cap; j += kTopkThreads) {
    oi[j] = 0;
    ov[j] = 0;
    ow[j] = 0.0f;
  }
  if (k == 0) {
    if (tid == 0) {
      mass[r] = 0.0f;
      if (counts) counts[r] = 0;
    }
    return;
  }

  // ---- 1. load
  float mx = -INFINITY, mn = INFINITY;
  {
    float xs[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int i = j * kTopkThreads + tid;
      xs[j] = (i < n) ? x[i] : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int i = j * kTopkThreads + tid;
      if (i < n) {
        sh.keys[i] = order_key(xs[j]);
        mx = fmaxf(mx, xs[j]);
        mn = fminf(mn, xs[j]);
      }
    }
  }
  for (int i = tid; i < kBins; i += kTopkThreads) (&sh.hist[0][0])[i] = 0;
  if (tid == 0) sh.ncand = 0;
  const float M = lds_block_max(mx, sh);
  mn = -lds_block_max(-mn, sh);
  // non-finite extremes collapse every key into bin 0 (the fallback then covers all)
  const float inv = (isfinite(M) && isfinite(mn) && M > mn) ? static_cast<float>(kBins) / (M - mn) : 0.0f;

  // ---- 2. normaliser and value histogram
  float z = 0.0f;
  uint32_t* lin = &sh.hist[0][0];  // one kBins-bin histogram (the sub-histograms are for the radix)
  for (int i = tid; i < n; i += kTopkThreads) {
    const float xi = key_value(sh.keys[i]);
    z += fast_exp2((xi - M) * kLog2e);
    atomicAdd(&lin[value_bin(xi, mn, inv)], 1u);
  }
  const float Z = lds_block_sum(z, sh);  // (its barriers also complete the histogram)
  {
    const int bin = kBins - 1 - tid;  // descending scan: thread t owns bin kBins-1-t
    const uint32_t h = lin[bin];
    uint32_t incl = h;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const uint32_t o = __shfl_up(incl, off, kWave);
      if (lane >= off) incl += o;
    }
    if (lane == 63) sh.cnt[0][w] = incl;
    __syncthreads();
    uint32_t base = 0;
    for (int q = 0; q < w; ++q) base += sh.cnt[0][q];
    const uint32_t above = base + incl - h;
    if (above < static_cast<uint32_t>(k) && above + h >= static_cast<uint32_t>(k)) {
      sh.sel_digit = static_cast<uint32_t>(bin);
      sh.bin_above = above;
    }
    __syncthreads();
  }
  const int bstar = static_cast<int>(sh.sel_digit);
  const int need_b = k - static_cast<int>(sh.bin_above);  // >= 1 keys of B* are selected

  // ---- 3. keys of the boundary bin -> (kth_key, kth_idx)
  for (int i = tid; i < n; i += kTopkThreads) {
    const uint32_t kk = sh.keys[i];
    if (value_bin(key_value(kk), mn, inv) == bstar) {
      const uint32_t slot = atomicAdd(&sh.ncand, 1u);
      if (slot < kCand) {
        sh.cand_key[slot] = kk;
        sh.cand_idx[slot] = static_cast<uint32_t>(i);
      }
    }
  }
  __syncthreads();
  const int m = static_cast<int>(sh.ncand);
  if (m <= kCand) {
    if (tid < m) {
      const uint32_t mk = sh.cand_key[tid], mi = sh.cand_idx[tid];
      int rank = 0;
      for (int u = 0; u < m; ++u) {
        const uint32_t uk = sh.cand_key[u], ui = sh.cand_idx[u];
        rank += (uk > mk || (uk == mk && ui < mi)) ? 1 : 0;
      }
      if (rank == need_b - 1) {
        sh.kth_key = mk;
        sh.kth_idx = mi;
      }
    }
  } else {
    // crowded bin (many equal or clustered scores): exact radix select within B*
    uint32_t prefix = 0, pmask = 0;
    int remaining = need_b;
    uint32_t* hist = &sh.hist[w & (kSubHist - 1)][0];
    for (int shift = 24; shift >= 0; shift -= 8) {
      for (int i = tid; i < kSubHist * 256; i += kTopkThreads) (&sh.hist[0][0])[i] = 0;
      __syncthreads();
      for (int i = tid; i < n; i += kTopkThreads) {
        const uint32_t kk = sh.keys[i];
        if ((kk & pmask) == prefix && value_bin(key_value(kk), mn, inv) == bstar)
          atomicAdd(&hist[(kk >> shift) & 0xFFu], 1u);
      }
      __syncthreads();
      if (tid < kWave) {
        uint32_t h[4];
        uint32_t local = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int bin = 255 - 4 * lane - e;
          h[e] = 0;
#pragma unroll
          for (int q = 0; q < kSubHist; ++q) h[e] += sh.hist[q][bin];
          local += h[e];
        }
        uint32_t incl = local;
#pragma unroll
        for (int off = 1; off < kWave; off <<= 1) {
          const uint32_t o = __shfl_up(incl, off, kWave);
          if (lane >= off) incl += o;
        }
        uint32_t above = incl - local;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (above < static_cast<uint32_t>(remaining) && above + h[e] >= static_cast<uint32_t>(remaining)) {
            sh.sel_digit = 255 - 4 * lane - e;
            sh.bin_above = above;
          }
          above += h[e];
        }
      }
      __syncthreads();
      prefix |= sh.sel_digit << shift;
      pmask |= 0xFFu << shift;
      remaining -= static_cast<int>(sh.bin_above);
      __syncthreads();
    }
    // the `remaining`-th key equal to `prefix` in index order is the k-th key
#pragma unroll 1
    for (int j = 0; j < kPer; ++j) {
      const int i = j * kTopkThreads + tid;
      const bool eq = i < n && sh.keys[i] == prefix;
      const uint64_t bal = __ballot(eq);
      if (lane == 0) sh.cnt[j][w] = static_cast<uint32_t>(__popcll(bal));
    }
    __syncthreads();
    prefix_counts(sh);
#pragma unroll 1
    for (int j = 0; j < kPer; ++j) {
      const int i = j * kTopkThreads + tid;
      const bool eq = i < n && sh.keys[i] == prefix;
      const uint64_t bal = __ballot(eq);
      const int rank = static_cast<int>(sh.cnt[j][w]) + __popcll(bal & lt_mask);
      if (eq && rank == remaining - 1) {
        sh.kth_key = prefix;
        sh.kth_idx = static_cast<uint32_t>(i);
      }
    }
  }
  __syncthreads();
  const uint32_t kth_key = sh.kth_key;
  const uint32_t kth_idx = sh.kth_idx;

  // ---- 4. selected keys in index order
#pragma unroll 1
  for (int j = 0; j < kPer; ++j) {
    const int i = j * kTopkThreads + tid;
    const uint32_t kk = i < n ? sh.keys[i] : 0u;
    const bool sel = i < n && (kk > kth_key || (kk == kth_key && static_cast<uint32_t>(i) <= kth_idx));
    const uint64_t bal = __ballot(sel);
    if (lane == 0) sh.cnt[j][w] = static_cast<uint32_t>(__popcll(bal));
  }
  __syncthreads();
  prefix_counts(sh);
  float msum = 0.0f;
  const float invZ = 1.0f / Z;
#pragma unroll 1
  for (int j = 0; j < kPer; ++j) {
    const int i = j * kTopkThreads + tid;
    const uint32_t kk = i < n ? sh.keys[i] : 0u;
    const bool sel = i < n && (kk > kth_key || (kk == kth_key && static_cast<uint32_t>(i) <= kth_idx));
    const uint64_t bal = __ballot(sel);
    const int pos = static_cast<int>(sh.cnt[j][w]) + __popcll(bal & lt_mask);
    if (sel && pos < cap) {
      const float wv = fast_exp2((key_value(kk) - M) * kLog2e) * invZ;
      oi[pos] = i;
      ov[pos] = 1;
      ow[pos] = wv;
      msum += wv;
    }
  }
  const float S = lds_block_sum(msum, sh);  // its barriers also order the weight writes
  const float invS = 1.0f / S;
  for (int j = tid; j < k; j += kTopkThreads) ow[j] *= invS;
  if (tid == 0) {
    mass[r] = S;
    if (counts) counts[r] = k;
  }
}

struct EligibleCand {
  const uint8_t* elig;
  int last;  // excluded index (forced), or -1
  __device__ bool operator()(int i) const { return i != last && (elig == nullptr || elig[i] != 0); }
};

__global__ __launch_bounds__(kTopkThreads) void select_tokens_kernel(const float* scores, int tokens, double fraction,
                                                                     const uint8_t* eligible, int force_last,
                                                                     uint8_t* mask, int32_t* positions,
                                                                     int32_t* counts, int32_t* error_flag) {
  __shared__ TopkShared sh;
  __shared__ int n_elig_sh;
  const int b = blockIdx.x;
  const float* x = scores + static_cast<int64_t>(b) * tokens;
  const uint8_t* el = eligible ? eligible + static_cast<int64_t>(b) * tokens : nullptr;
  uint8_t* om = mask + static_cast<int64_t>(b) * tokens;
  int32_t* op = positions ? positions + static_cast<int64_t>(b) * tokens : nullptr;
  for (int i = threadIdx.x; i < tokens; i += kTopkThreads) {
    om[i] = 0;
    if (op) op[i] = 0;
  }
  const int last = tokens - 1;
  const bool forced = force_last != 0;
  if (threadIdx.x == 0) n_elig_sh = 0;
  __syncthreads();
  int cnt = 0;
  for (int i = threadIdx.x; i < tokens; i += kTopkThreads) cnt += (el == nullptr || el[i] != 0) ? 1 : 0;
  atomicAdd(&n_elig_sh, cnt);
  __syncthreads();
  const int n_elig = n_elig_sh;
  if (n_elig == 0 || (forced && el != nullptr && el[last] == 0)) {
    if (threadIdx.x == 0) {
      if (error_flag) atomicExch(error_flag, 1);
      if (counts) counts[b] = 0;
    }
    return;
  }
  const double want = ceil(static_cast<double>(tokens) * fraction);
  const int budget = static_cast<int>(want < 1.0 ? 1.0 : want);
  const int count = min(budget, n_elig);  // candidates + forced == n_elig
  const int remaining = count - (forced ? 1 : 0);
  __syncthreads();
  int selected = 0;
  if (remaining > 0) {
    const EligibleCand cand{el, forced ? last : -1};
    uint32_t kth;
    int need;
    radix_select(x, tokens, remaining, cand, sh, &kth, &need);
    // positions are written after the forced token is merged in, below
    selected = compact_selected(x, tokens, kth, need, cand, sh, [&](int i, int) { om[i] = 1; });
  }
  __threadfence_block();
  __syncthreads();
  if (forced && threadIdx.x == 0) om[last] = 1;
  __threadfence_block();
  __syncthreads();
  if (op) {
    // ascending positions of the final mask
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    int out_base = 0;
    for (int base = 0; base < tokens; base += kTopkThreads) {
      const int i = base + threadIdx.x;
      const bool s = i < tokens && om[i] != 0;
      const uint64_t bal = __ballot(s);
      if (lane == 0) sh.wave_cnt[w] = static_cast<uint32_t>(__popcll(bal));
      __syncthreads();
      int pos = out_base + __popcll(bal & lt_mask);
      int tot = 0;
      for (int j = 0; j < kTopkWaves; ++j) {
        if (j < w) pos += static_cast<int>(sh.wave_cnt[j]);
        tot += static_cast<int>(sh.wave_cnt[j]);
      }
      if (s) op[pos] = i;
      out_base += tot;
      __syncthreads();
    }
  }
  if (threadIdx.x == 0 && counts) counts[b] = selected + (forced ? 1 : 0);
}

}  // namespace
}  // namespace fl

extern "C" int32_t fl_decode_topk(const float* scores, int64_t scores_stride, int32_t rows, const int32_t* n_keys,
                                  int32_t rows_per_count, double fraction, int32_t capacity, int32_t* indices,
                                  uint8_t* valid, float* mass, float* weights, int32_t* counts, void* stream) {
  using namespace fl;
  clear_error();
  FL_REQUIRE(scores && n_keys && indices && valid && mass && weights, "fl_decode_topk: null pointer");
  FL_REQUIRE(rows >= 0 && rows_per_count > 0 && capacity > 0, "fl_decode_topk: bad rows/rows_per_count/capacity");
  FL_REQUIRE(fraction > 0.0 && fraction <= 1.0, "fl_decode_topk: fraction must be in (0, 1]");
  FL_REQUIRE(scores_stride > 0, "fl_decode_topk: bad stride");
  if (rows == 0) return FL_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(rows), block(kTopkThreads);  // block: fallback kernel
  // the stride bounds every row's key count: rows that fit in LDS take the one-read kernel
  if (scores_stride <= kLdsKeys)
    hipLaunchKernelGGL(decode_topk_lds_kernel, grid, block, 0, st, scores, scores_stride, n_keys, rows_per_count,
                       fraction, capacity, indices, valid, mass, weights, counts);
  else
    hipLaunchKernelGGL(decode_topk_kernel, grid, block, 0, st, scores, scores_stride, n_keys, rows_per_count,
                       fraction, capacity, indices, valid, mass, weights, counts);
  FL_LAUNCH_CHECK("fl_decode_topk");
  return FL_OK;
}

extern "C" int32_t fl_select_tokens(const float* scores, int32_t batch, int32_t tokens, double fraction,
                                    const uint8_t* eligible, int32_t force_last, uint8_t* mask, int32_t* positions,
                                    int32_t* counts, int32_t* error_flag, void* stream) {
  using namespace fl;
  clear_error();
  FL_REQUIRE(scores && mask, "fl_select_tokens: null scores/mask");
  FL_REQUIRE(batch >= 0 && tokens > 0, "fl_select_tokens: scores must have shape [batch, tokens>0]");
  FL_REQUIRE(fraction > 0.0 && fraction <= 1.0, "fl_select_tokens: fraction must satisfy 0 < fraction <= 1");
  if (batch == 0) return FL_OK;
  hipLaunchKernelGGL(select_tokens_kernel, dim3(batch), dim3(kTopkThreads), 0, static_cast<hipStream_t>(stream),
                     scores, tokens, fraction, eligible, force_last, mask, positions, counts, error_flag);
  FL_LAUNCH_CHECK("fl_select_tokens");
  return FL_OK;
}
