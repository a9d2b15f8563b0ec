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
// unsigned keys.  Decode rows of up to 35K keys are held in registers and selected in
// one read (decode_topk_resident_kernel).  Longer rows and the prefill token selection
// re-read the row (it stays in L2): four 8-bit histogram passes (LDS atomics) find the
// k-th largest key K* and how many keys equal to K* to take, then a final pass walks the
// row in index order, takes every key > K* and the first `need` keys == K*
// (ballot/popcount ranks), and writes the selected indices in ascending order.
#include "dense_layout.h"
#include "internal.h"

namespace fl {
namespace {

constexpr int kTopkThreads = 1024;
constexpr int kTopkWaves = kTopkThreads / kWave;
// Slot order of a row's keys over a workgroup: key q*4096 + 4t + e is thread t's slot
// 4q + e, so a thread reads 16 contiguous bytes per quad chunk q.
constexpr int kQuadChunk = 4 * kTopkThreads;

// Order-preserving unsigned key of a score.  -0.0 takes the key of +0.0 (they compare
// equal, so the lower index wins their tie, as in torch.topk and a stable sort): adding
// +0.0 maps -0.0 to +0.0 and leaves every other value (NaN included) as it is.
__device__ __forceinline__ uint32_t order_key(float f) {
  const uint32_t u = __float_as_uint(f + 0.0f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
// NaN or +-inf (flashloop/selection.py:78-79 rejects such weights)
__device__ __forceinline__ bool non_finite(float f) { return !(fabsf(f) <= 3.402823466e38f); }
__device__ __forceinline__ float key_value(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k ^ 0x80000000u) : ~k);
}

// ---- Ranking key of the decode selection: the fp32 softmax weight.
// flashloop/engine.py:439-453 ranks w = softmax(logits, dtype=float32) with torch.topk
// (selection.py:85 likewise), so distinct logits whose weights round to one fp32 value tie
// there -- e.g. every key whose weight underflows to 0 in a peaked row -- and the tie goes
// to the lower index.  The kernels rank the same image:
//   e = softmax_exp(RN(x - max)),  Z = row_weight_sum(e),  w = RN(e * RN(1/Z)),
// key = bits(w) + 1 (w >= 0, so the bits order like the values; key 0 marks padding).
// softmax_exp uses IEEE fma/mul only and Z has a fixed summation order, so every bit of
// w is reproducible on the CPU.  This file is compiled with -ffp-contract=off.
constexpr float kInvLn2 = 0x1.715476p+0f;   // RN(1/ln 2)
constexpr float kLn2Hi = 0x1.62e430p-1f;    // RN(ln 2)
constexpr float kLn2Lo = -0x1.05c610p-29f;  // RN(ln 2 - kLn2Hi)

// exp(d) for d <= 0 (d = -inf gives 0): Cody-Waite reduction d = n ln2 + r, |r| <= ln2/2,
// the degree-7 Taylor polynomial of e^r by Horner (truncation 5e-9 relative), and the
// scale 2^n applied as an exact multiply by 2^(n+64) and a rounding multiply by 2^-64,
// so a result in the subnormal range is rounded once.  Within ~2 ulp of exp.
__device__ __forceinline__ float softmax_exp(float d) {
  d = fmaxf(d, -112.0f);  // exp(-112) rounds to 0 as every smaller argument does
  const float n = rintf(d * kInvLn2);
  float r = fmaf(n, -kLn2Hi, d);
  r = fmaf(n, -kLn2Lo, r);
  float p = 0x1.a01a02p-13f;      // 1/7!
  p = fmaf(p, r, 0x1.6c16c2p-10f);  // 1/6!
  p = fmaf(p, r, 0x1.111112p-7f);   // 1/5!
  p = fmaf(p, r, 0x1.555556p-5f);   // 1/4!
  p = fmaf(p, r, 0x1.555556p-3f);   // 1/3!
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  const float up = __uint_as_float(static_cast<uint32_t>(static_cast<int>(n) + 64 + 127) << 23);  // 2^(n+64)
  const float e = p * up;
  return e * 0x1p-64f;
}

// w = RN(e * invZ) as a ranking key (>= 1)
__device__ __forceinline__ uint32_t weight_key(float e, float invZ) { return __float_as_uint(e * invZ) + 1u; }
__device__ __forceinline__ float key_weight(uint32_t key) { return __uint_as_float(key - 1u); }
// key of a row that holds NaN or +inf (its softmax is NaN throughout): the score order,
// -inf ranked as -FLT_MAX, every key >= 1
constexpr uint32_t kScoreKeyFloor = 0x00800000u;  // order_key(-FLT_MAX)
__device__ __forceinline__ uint32_t score_key(float x) { return max(order_key(x), kScoreKeyFloor); }

// Sum over a wave in a fixed order: pairs at lane distance 32, 16, ..., 1 (every lane ends
// with the same bits: a + b and b + a round alike).
__device__ __forceinline__ float wave_sum_fixed(float v) {
#pragma unroll
  for (int off = kWave / 2; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// Sum over the workgroup in a fixed order: wave_sum_fixed, then the 16 wave sums in wave
// order.
template <typename Sh>
__device__ float res_block_sum_fixed(float v, Sh& sh) {
  v = wave_sum_fixed(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh.red[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = sh.red[0];
#pragma unroll
  for (int i = 1; i < kTopkWaves; ++i) r += sh.red[i];
  return r;
}

struct TopkShared {
  uint32_t hist[256];
  uint32_t wave_cnt[kTopkWaves];
  uint32_t wave_cnt2[kTopkWaves];
  float red[kTopkWaves];
  uint32_t sel_prefix;
  uint32_t sel_remaining;
  uint32_t bin_above;
  uint32_t nonfin;
  uint32_t has_nan;
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

// Radix-select the k-th largest candidate key (key(i): the ranking key of index i) of the
// row.  On return (all threads): *kth = K*, *need = number of keys equal to K* to take
// (taking lowest indices first).
template <typename Key, typename Cand>
__device__ void radix_select(Key key_of, int n, int k, Cand cand, TopkShared& sh, uint32_t* kth, int* need) {
  uint32_t prefix = 0, mask = 0;
  int remaining = k;
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int i = threadIdx.x; i < 256; i += kTopkThreads) sh.hist[i] = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += kTopkThreads) {
      if (!cand(i)) continue;
      const uint32_t key = key_of(i);
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

// Walk the row in index order; call emit(i, out_pos, key) for every selected candidate.
// Returns the number selected.
template <typename Key, typename Cand, typename Emit>
__device__ int compact_selected(Key key_of, int n, uint32_t kth, int need, Cand cand, TopkShared& sh, Emit emit) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  int eq_base = 0, out_base = 0;
  for (int base = 0; base < n; base += kTopkThreads) {
    const int i = base + threadIdx.x;
    bool gt = false, eq = false;
    uint32_t key = 0;
    if (i < n && cand(i)) {
      key = key_of(i);
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
    if (sel) emit(i, pos, key);
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
                                                                   int32_t* counts, int32_t* nonfinite) {
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
      if (nonfinite) nonfinite[r] = 0;
    }
    return;
  }
  // softmax statistics of the row (flashloop/engine.py:440-442) and its non-finite scores
  if (threadIdx.x == 0) {
    sh.nonfin = 0;
    sh.has_nan = 0;
  }
  float mx = -INFINITY;
  uint32_t nf = 0, amax = 0;
  for (int i = threadIdx.x; i < n; i += kTopkThreads) {
    const float xi = x[i];
    mx = fmaxf(mx, xi);
    amax = max(amax, __float_as_uint(xi) & 0x7FFFFFFFu);
    nf += non_finite(xi) ? 1u : 0u;
  }
  const float M = block_max(mx, sh);  // (its barriers order the counter's reset)
  if (nf) atomicAdd(&sh.nonfin, nf);
  if (amax > 0x7F800000u) sh.has_nan = 1u;  // |x|'s bits above inf's: a NaN
  __syncthreads();
  const bool weighted = sh.has_nan == 0u && M > -INFINITY && M < INFINITY;
  // the same weight image and summation order as the register-resident kernel: thread t
  // sums indices q*4096 + 4t + e in (q, e) order, then the fixed-order block sum
  float invZ = 0.0f;
  if (weighted) {
    float z = 0.0f;
    for (int base = 4 * threadIdx.x; base < n; base += kQuadChunk)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (base + e < n) z += softmax_exp(x[base + e] - M);
    invZ = 1.0f / res_block_sum_fixed(z, sh);
  }
  const auto key_of = [&](int i) {
    return weighted ? weight_key(softmax_exp(x[i] - M), invZ) : score_key(x[i]);
  };

  uint32_t kth;
  int need;
  radix_select(key_of, n, k, AllCand{}, sh, &kth, &need);
  float msum = 0.0f;
  compact_selected(key_of, n, kth, need, AllCand{}, sh, [&](int i, int pos, uint32_t key) {
    const float w = weighted ? key_weight(key) : NAN;
    oi[pos] = i;
    ov[pos] = 1;
    ow[pos] = w;
    msum += w;
  });
  const float S = block_sum(msum, sh);
  __threadfence_block();
  __syncthreads();
  for (int j = threadIdx.x; j < cap; j += kTopkThreads) {
    if (j < k) {
      ow[j] = ow[j] / S;  // selected_global / mass (engine.py:492)
    } else {
      oi[j] = 0;
      ov[j] = 0;
      ow[j] = 0.0f;
    }
  }
  if (threadIdx.x == 0) {
    mass[r] = S;
    if (counts) counts[r] = k;
    if (nonfinite) nonfinite[r] = static_cast<int32_t>(sh.nonfin);
  }
}

// Register-resident variant for rows of at most kResKeys keys and k <= kSelLds: thread t
// holds keys q*4096 + 4t + e (slot 4q + e) in registers for the whole kernel, so no pass
// after the load re-reads the row.  The passes are VALU-bound (one row per CU), so each
// is kept to a few instructions per key:
//   1. load (one dwordx4 per quad, all issued first), row max and min;
//   2. the keys: the fp32 softmax weight image (or the score order in a row without
//      finite weights);
//   3. a histogram over kBins key-linear bins -- the bin is a non-decreasing function of
//      the key, so the k-th largest key lies in the bin B* where the count from the top
//      reaches k, and every key of a higher bin is larger;
//   4. per (quad chunk, wave) ballot counts of the keys above B*, and the keys of B* (a
//      few dozen for smooth score distributions) compacted into an LDS list, ranked there
//      by (key desc, index asc): that fixes the k-th key (kth_key, kth_idx) and adds the
//      selected keys of B* to their (chunk, wave) counts -- a bin too crowded for the
//      list falls back to an exact radix select restricted to B* and a counting pass;
//   5. one prefix scan of the counts, then each lane stores its selected (index, key) at
//      its offset in an LDS list, which is therefore in index order;
//   6. the k list entries get their softmax weights and are written out coalesced.
constexpr int kPer = 36;  // most keys per thread (rows of up to kResKeys keys); a multiple of 4
constexpr int kResKeys = kPer * kTopkThreads;
constexpr int kSelLds = 8 * kTopkThreads;  // selected-list capacity of the resident kernel
constexpr int kSelPer = kSelLds / kTopkThreads;
constexpr int kSubHist = 4;
constexpr int kBins = kSubHist * 256;  // value-linear bins of the boundary search (one per thread)
constexpr int kCand = 512;             // boundary-bin list capacity
static_assert(kBins == kTopkThreads, "one boundary bin per thread");

__device__ __forceinline__ uint64_t ballot64(bool p) { return __builtin_amdgcn_ballot_w64(p); }

struct ResShared {
  uint32_t hist[kSubHist][256];
  uint32_t cnt[kPer][kTopkWaves];  // per (chunk, wave) counts, then their exclusive prefix
  uint32_t cand_key[kCand];
  uint32_t cand_idx[kCand];
  uint32_t cand_rank[kCand];
  uint32_t sel_idx[kSelLds];
  uint32_t sel_key[kSelLds];
  uint16_t bin[kPer][kTopkThreads];  // value bin of each key (pass 2), read by pass 3
  float red[kTopkWaves];
  float red2[kTopkWaves];
  float red3[kTopkWaves];
  uint32_t sel_digit;
  uint32_t bin_above;
  uint32_t ncand;
  uint32_t kth_key;
  uint32_t kth_idx;
  uint32_t total;
  uint32_t nonfin;
};

__device__ float res_block_max(float v, ResShared& sh) {
  v = wave_max(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh.red[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = sh.red[0];
#pragma unroll
  for (int i = 1; i < kTopkWaves; ++i) r = fmaxf(r, sh.red[i]);
  return r;
}

// max over the workgroup of a, of b and of c, in one exchange
__device__ float3 res_block_max3(float a, float b, float c, ResShared& sh) {
  a = wave_max(a);
  b = wave_max(b);
  c = wave_max(c);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) {
    sh.red[threadIdx.x >> 6] = a;
    sh.red2[threadIdx.x >> 6] = b;
    sh.red3[threadIdx.x >> 6] = c;
  }
  __syncthreads();
  float3 r = make_float3(sh.red[0], sh.red2[0], sh.red3[0]);
#pragma unroll
  for (int i = 1; i < kTopkWaves; ++i) {
    r.x = fmaxf(r.x, sh.red[i]);
    r.y = fmaxf(r.y, sh.red2[i]);
    r.z = fmaxf(r.z, sh.red3[i]);
  }
  return r;
}

__device__ float res_block_sum(float v, ResShared& sh) {
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
template <int PER>
__device__ uint32_t prefix_counts(ResShared& sh) {
  if (threadIdx.x < kWave) {
    const int lane = threadIdx.x;
    constexpr int kN = PER * kTopkWaves;
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
    if (lane == kWave - 1) sh.total = incl;
  }
  __syncthreads();
  return sh.total;
}

struct TopkArgs {
  const float* scores;
  int64_t stride;
  double fraction;
  int cap;
  int32_t* indices;
  uint8_t* valid;
  float* mass;
  float* weights;
  int32_t* counts;
  int32_t* nonfinite;
};

// Top-k of row r = blockIdx.x (key_count(r) keys) by one 1024-thread workgroup.  Slot
// j = 4q + e of thread t holds key q*4096 + 4t + e: each thread loads 16 bytes per quad
// chunk (one dwordx4 load per 4 keys; dword loads had made the load pass 4x longer).
template <int PER, typename KeyCount>
__device__ __forceinline__ void topk_resident_row(ResShared& sh, KeyCount key_count, const float* scores, int64_t stride,
                                                  double fraction, int cap, int32_t* indices, uint8_t* valid,
                                                  float* mass, float* weights, int32_t* counts, int32_t* nonfinite) {
  static_assert(PER % 4 == 0 && PER <= kPer, "keys per thread: whole quads within the LDS arrays");
  constexpr int Q = PER / 4;
  const int r = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const float* x = scores + static_cast<int64_t>(r) * stride;
  int n = min(key_count(r), static_cast<int>(min<int64_t>(stride, 0x7fffffff)));
  n = min(n, PER * kTopkThreads);
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
  if (k > kSelLds) k = kSelLds;  // the host routes rows that could exceed it elsewhere
  for (int j = k + tid; j < cap; j += kTopkThreads) {
    oi[j] = 0;
    ov[j] = 0;
    ow[j] = 0.0f;
  }
  if (k == 0) {
    if (tid == 0) {
      mass[r] = 0.0f;
      if (counts) counts[r] = 0;
      if (nonfinite) nonfinite[r] = 0;
    }
    return;
  }
  const auto index_of = [&](int j) { return (j >> 2) * kQuadChunk + 4 * tid + (j & 3); };
  // Quad chunk q holds keys below n (row-uniform).  In the shorter-row instantiations
  // (ragged batches put rows of any length in one) the exp and histogram passes skip the
  // chunks past n: cfg2's select launch 44.3 -> 41.4 us.  The 36-key instantiation keeps
  // branch-free passes: a branch per chunk there cost its 32,769-key rows 0.5-1 us.
  constexpr bool kSkipDead = PER <= 20;
  const auto quad_live = [&](int q) { return !kSkipDead || q * kQuadChunk < n; };

  // ---- 1. load, row max and min, and what kinds of non-finite score the row holds (the
  // max of |x|'s bits: above inf's bits is a NaN).  Every load is issued before the first
  // use: bounds-checked buffer loads (keys past n read as zero, then replaced by -inf),
  // 16 bytes per quad when the row is 16-byte aligned; the one lane whose quad straddles
  // n reloads its keys.
  uint32_t kr[PER];  // the score bits, then e's bits, then the ranking key (0 = padding)
  float mx = -INFINITY, mn = INFINITY;
  uint32_t amax = 0;
  if (tid == 0) sh.nonfin = 0;
  {
    const __amdgpu_buffer_rsrc_t res =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(x), 0, n * static_cast<int>(sizeof(float)), 0x00020000);
    float xs[PER];
    if ((reinterpret_cast<uintptr_t>(x) & 15u) == 0) {  // (row-uniform) 16-byte aligned row
#pragma unroll
      for (int q = 0; q < Q; ++q) {
        const float4 t4 = __builtin_bit_cast(
            float4, __builtin_amdgcn_raw_buffer_load_b128(res, (q * kQuadChunk + 4 * tid) * 4, 0, 0));
        xs[4 * q] = t4.x;
        xs[4 * q + 1] = t4.y;
        xs[4 * q + 2] = t4.z;
        xs[4 * q + 3] = t4.w;
      }
    } else {
#pragma unroll
      for (int j = 0; j < PER; ++j)
        xs[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(res, index_of(j) * 4, 0, 0));
    }
    const int qs = (n - 1) / kQuadChunk, ts = ((n - 1) % kQuadChunk) >> 2;  // the straddling quad
    if ((n & 3) != 0 && tid == ts) {
#pragma unroll
      for (int q = 0; q < Q; ++q)
        if (q == qs)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int i = q * kQuadChunk + 4 * tid + e;
            if (i < n) xs[4 * q + e] = x[i];
          }
    }
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const bool in = index_of(j) < n;
      xs[j] = in ? xs[j] : -INFINITY;
      kr[j] = __float_as_uint(xs[j]);
      amax = max(amax, in ? kr[j] & 0x7FFFFFFFu : 0u);
      mx = fmaxf(mx, xs[j]);
      mn = fminf(mn, in ? xs[j] : INFINITY);
    }
  }
  for (int i = tid; i < kBins; i += kTopkThreads) (&sh.hist[0][0])[i] = 0;
  if (tid == 0) sh.ncand = 0;
  // flag 2: a NaN; flag 1: an infinity
  const float flag = amax > 0x7F800000u ? 2.0f : (amax == 0x7F800000u ? 1.0f : 0.0f);
  const float3 ext = res_block_max3(mx, -mn, flag, sh);  // (its barriers order the reset)
  const float M = ext.x;
  mn = -ext.y;
  // softmax weights exist unless the row holds a NaN or +inf, or only -inf (then torch's
  // fp32 softmax is NaN throughout and the score order ranks instead)
  const bool weighted = ext.z < 2.0f && M > -INFINITY && M < INFINITY;
  const bool badrow = ext.z != 0.0f;  // some score may be non-finite: counted below

  // ---- 2. the weight image (weighted rows) or the score order, as keys.  Thread t sums
  // its e in slot order, then the fixed-order block sum.
  float invZ = 0.0f;
  uint32_t kmin = kScoreKeyFloor, shift = 31u, binmax = 0u;  // a score-ordered row: one bin
  if (weighted) {
    float z = 0.0f;  // (padding's -inf adds +0)
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      if (!quad_live(q)) continue;  // padding only: e = 0 adds nothing
#pragma unroll
      for (int j = 4 * q; j < 4 * q + 4; ++j) {
        const float e = softmax_exp(__uint_as_float(kr[j]) - M);
        z += e;
        kr[j] = __float_as_uint(e);
      }
    }
    const float Z = res_block_sum_fixed(z, sh);
    invZ = 1.0f / Z;
#pragma unroll
    for (int j = 0; j < PER; ++j) kr[j] = index_of(j) < n ? weight_key(__uint_as_float(kr[j]), invZ) : 0u;
    // keys lie in [key(min score), key(max score) = bits(invZ) + 1]; bins of 2^shift keys
    kmin = weight_key(softmax_exp(mn - M), invZ);
    const uint32_t span = max(__float_as_uint(invZ) + 1u, kmin) - kmin;
    shift = span < static_cast<uint32_t>(kBins) ? 0u : 32u - static_cast<uint32_t>(__clz(span)) - 10u;
    binmax = kBins - 1;
  } else {
#pragma unroll
    for (int j = 0; j < PER; ++j) kr[j] = index_of(j) < n ? score_key(__uint_as_float(kr[j])) : 0u;
  }

  // ---- 3. histogram: bin(key) is non-decreasing in the key.  Padding is not counted: a
  // row's padding all on one bin would serialise its LDS atomics.
  uint32_t* lin = &sh.hist[0][0];  // one kBins-bin histogram (the sub-histograms are for the radix)
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    if (!quad_live(q)) continue;  // bins of dead chunks are never read (passes 4-5 skip them)
#pragma unroll
    for (int j = 4 * q; j < 4 * q + 4; ++j) {
      const int b = static_cast<int>(min(static_cast<uint32_t>(max(static_cast<int>(kr[j] - kmin), 0)) >> shift, binmax));
      sh.bin[j][tid] = static_cast<uint16_t>(b);
      if (kr[j] != 0u) atomicAdd(&lin[b], 1u);
    }
  }
  __syncthreads();  // the histogram is complete
  // Only a row holding a non-finite score (the same decision in every thread) counts
  // them, re-reading the row.
  if (badrow) {
    uint32_t c = 0;
    for (int i = tid; i < n; i += kTopkThreads) c += non_finite(x[i]) ? 1u : 0u;
    if (c) atomicAdd(&sh.nonfin, c);
  }
  {
    const int bin = kBins - 1 - tid;  // descending scan: thread t owns bin kBins-1-t
    const uint32_t h = lin[bin];
    uint32_t incl = h;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      const uint32_t u = __shfl_up(incl, o, kWave);
      if (lane >= o) incl += u;
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

  // ---- 4. counts of the keys above B* per (quad chunk, wave); keys of B* -> LDS list
  // (one LDS atomic per wave)
  uint32_t cnt_lane = 0;  // lane q: this wave's count of quad chunk q
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    uint32_t c = 0;
    if (q * kQuadChunk >= n) continue;  // (row-uniform) a chunk past the row's keys
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int j = 4 * q + e;
      const int b = sh.bin[j][tid];
      c += static_cast<uint32_t>(__popcll(ballot64(b > bstar)));
      const bool in_b = b == bstar && kr[j] != 0u;
      const uint64_t bal_b = ballot64(in_b);
      if (bal_b != 0ull) {
        uint32_t base = 0;
        if (lane == 0) base = atomicAdd(&sh.ncand, static_cast<uint32_t>(__popcll(bal_b)));
        base = __shfl(base, 0, kWave);
        const uint32_t slot = base + static_cast<uint32_t>(__popcll(bal_b & lt_mask));
        if (in_b && slot < kCand) {
          sh.cand_key[slot] = kr[j];
          sh.cand_idx[slot] = static_cast<uint32_t>(index_of(j));
        }
      }
    }
    cnt_lane = lane == q ? c : cnt_lane;
  }
  if (lane < Q) sh.cnt[lane][w] = cnt_lane;
  if (tid < kCand) sh.cand_rank[tid] = 0;
  __syncthreads();
  // (quad chunk, wave) of key index i
  const auto chunk_of = [](uint32_t i) { return i / kQuadChunk; };
  const auto wave_of = [](uint32_t i) { return ((i % kQuadChunk) >> 2) / kWave; };
  const int m = static_cast<int>(sh.ncand);
  if (m <= kCand) {
    // rank of each candidate = how many candidates precede it in (key desc, index asc)
    // order.  The m x m comparisons are spread over all waves: wave w compares the 64
    // candidates of block w % nb against slice w / nb of the list.
    const int nb = (m + kWave - 1) / kWave;  // <= 8
    const int slices = kTopkWaves / nb;
    const int cb = w % nb, sl = w / nb;
    if (sl < slices) {
      const int c = cb * kWave + lane;
      const int chunk = (m + slices - 1) / slices;
      const int u0 = sl * chunk, u1 = min(m, u0 + chunk);
      const uint32_t mk = c < m ? sh.cand_key[c] : 0u, mi = c < m ? sh.cand_idx[c] : 0u;
      uint32_t rank = 0;
#pragma unroll 4
      for (int u = u0; u < u1; ++u) {
        const uint32_t uk = sh.cand_key[u], ui = sh.cand_idx[u];
        rank += (uk > mk || (uk == mk && ui < mi)) ? 1u : 0u;
      }
      if (c < m && rank) atomicAdd(&sh.cand_rank[c], rank);
    }
    __syncthreads();
    // the need_b best are selected and join their (chunk, wave) count
    if (tid < m) {
      const uint32_t mi = sh.cand_idx[tid];
      const int rank = static_cast<int>(sh.cand_rank[tid]);
      if (rank < need_b) atomicAdd(&sh.cnt[chunk_of(mi)][wave_of(mi)], 1u);
      if (rank == need_b - 1) {
        sh.kth_key = sh.cand_key[tid];
        sh.kth_idx = mi;
      }
    }
    __syncthreads();
  } else {
    // crowded bin (many equal or clustered keys): exact radix select within B*
    uint32_t prefix = 0, pmask = 0;
    int remaining = need_b;
    uint32_t* hist = &sh.hist[w & (kSubHist - 1)][0];
    for (int shift8 = 24; shift8 >= 0; shift8 -= 8) {
      for (int i = tid; i < kSubHist * 256; i += kTopkThreads) (&sh.hist[0][0])[i] = 0;
      __syncthreads();
#pragma unroll
      for (int j = 0; j < PER; ++j) {
        const uint32_t kk = kr[j];
        if (kk != 0u && (kk & pmask) == prefix && static_cast<int>(sh.bin[j][tid]) == bstar)
          atomicAdd(&hist[(kk >> shift8) & 0xFFu], 1u);
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
          for (int qh = 0; qh < kSubHist; ++qh) h[e] += sh.hist[qh][bin];
          local += h[e];
        }
        uint32_t incl = local;
#pragma unroll
        for (int o = 1; o < kWave; o <<= 1) {
          const uint32_t u = __shfl_up(incl, o, kWave);
          if (lane >= o) incl += u;
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
      prefix |= sh.sel_digit << shift8;
      pmask |= 0xFFu << shift8;
      remaining -= static_cast<int>(sh.bin_above);
      __syncthreads();
    }
    // the `remaining`-th key equal to `prefix` in index order is the k-th key
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      uint32_t c = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) c += static_cast<uint32_t>(__popcll(ballot64(kr[4 * q + e] == prefix)));
      if (lane == 0) sh.cnt[q][w] = c;
    }
    __syncthreads();
    prefix_counts<Q>(sh);
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      uint64_t bal[4];
      uint32_t before = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        bal[e] = ballot64(kr[4 * q + e] == prefix);
        before += static_cast<uint32_t>(__popcll(bal[e] & lt_mask));
      }
      int rank = static_cast<int>(sh.cnt[q][w] + before);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (kr[4 * q + e] == prefix) {
          if (rank == remaining - 1) {
            sh.kth_key = prefix;
            sh.kth_idx = static_cast<uint32_t>(index_of(4 * q + e));
          }
          ++rank;
        }
      }
    }
    __syncthreads();
    const uint32_t kk0 = sh.kth_key, ki0 = sh.kth_idx;
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      uint32_t c = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t kk = kr[4 * q + e];
        const bool sel = kk > kk0 || (kk == kk0 && static_cast<uint32_t>(index_of(4 * q + e)) <= ki0);
        c += static_cast<uint32_t>(__popcll(ballot64(sel)));
      }
      if (lane == 0) sh.cnt[q][w] = c;
    }
    __syncthreads();
  }
  const uint32_t kth_key = sh.kth_key;
  const uint32_t kth_idx = sh.kth_idx;
  prefix_counts<Q>(sh);  // (its barrier also publishes the counts to every wave)

  // ---- 5. selected (index, key) pairs into the LDS list, in index order: the offset of
  // (chunk q, wave w), then the selected keys of the lower lanes, then this lane's own
  const uint32_t base_lane = lane < Q ? sh.cnt[lane][w] : 0u;  // lane q: offset of chunk q
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    if (q * kQuadChunk >= n) continue;  // (row-uniform) no key of this chunk is selected
    bool sel[4];
    uint32_t before = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t kk = kr[4 * q + e];
      sel[e] = kk > kth_key || (kk == kth_key && static_cast<uint32_t>(index_of(4 * q + e)) <= kth_idx);
      before += static_cast<uint32_t>(__popcll(ballot64(sel[e]) & lt_mask));
    }
    int pos = static_cast<int>(__builtin_amdgcn_readlane(base_lane, q) + before);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (sel[e]) {
        if (pos < k) {
          sh.sel_idx[pos] = static_cast<uint32_t>(index_of(4 * q + e));
          sh.sel_key[pos] = kr[4 * q + e];
        }
        ++pos;
      }
    }
  }
  __syncthreads();

  // ---- 6. weights of the k selected keys, coalesced output
  // (a score-ordered row has no finite softmax: its weights and mass are NaN, as torch's are)
  float wv[kSelPer];
  float msum = 0.0f;
#pragma unroll
  for (int e = 0; e < kSelPer; ++e) {
    const int p = e * kTopkThreads + tid;
    wv[e] = 0.0f;
    if (p < k) {
      wv[e] = weighted ? key_weight(sh.sel_key[p]) : NAN;
      msum += wv[e];
    }
  }
  const float S = res_block_sum(msum, sh);
#pragma unroll
  for (int e = 0; e < kSelPer; ++e) {
    const int p = e * kTopkThreads + tid;
    if (p < k) {
      oi[p] = static_cast<int32_t>(sh.sel_idx[p]);
      ov[p] = 1;
      ow[p] = wv[e] / S;  // selected_global / mass (engine.py:492)
    }
  }
  if (tid == 0) {
    mass[r] = S;
    if (counts) counts[r] = k;
    if (nonfinite) nonfinite[r] = static_cast<int32_t>(sh.nonfin);
  }
}

template <int PER>
__global__ __launch_bounds__(kTopkThreads) void decode_topk_resident_kernel(const float* scores, int64_t stride,
                                                                            const int32_t* n_keys, int rows_per_count,
                                                                            double fraction, int cap, int32_t* indices,
                                                                            uint8_t* valid, float* mass, float* weights,
                                                                            int32_t* counts, int32_t* nonfinite) {
  __shared__ ResShared sh;
  topk_resident_row<PER>(
      sh, [&](int r) { return n_keys[r / rows_per_count]; }, scores, stride, fraction, cap, indices, valid, mass,
      weights, counts, nonfinite);
}

// The loop-2 top-k and the merge of the dense reader's rows in one launch: workgroups
// [0, B*H) select the keys of one row each (a row's key count is its packed prefix + tail +
// the current token, read from the cache view), workgroups [B*H, 2*B*H) merge one row's
// partials each.  The two halves are independent (both read only what the reader wrote),
// and the top-k's one-workgroup-per-row grid leaves half of the CUs free for the merges.
union SelectMergeLds {
  ResShared t;
  reader::DenseMergeLds m;
};

template <int PER>
__global__ __launch_bounds__(kTopkThreads) void select_merge_kernel(TopkArgs A, fl_cache_view v, const float* ws, int W,
                                                                    float* out) {
  __shared__ SelectMergeLds L;
  const int rows = v.batch * v.heads;
  if (static_cast<int>(blockIdx.x) < rows) {
    // row r's keys: its packed prefix, its tail and the current token (what the reader wrote)
    const auto key_count = [&](int r) {
      const int b = r / v.heads;
      return reader::row_groups(v, b) * kGroup + min(max(v.tail_tokens[b], 0), v.tail_capacity) + 1;
    };
    topk_resident_row<PER>(L.t, key_count, A.scores, A.stride, A.fraction, A.cap, A.indices, A.valid, A.mass,
                           A.weights, A.counts, A.nonfinite);
    return;
  }
  // the merge uses the first kMergeThreads threads; the other waves leave (a workgroup
  // barrier waits only for waves that have not ended)
  if (threadIdx.x >= reader::kMergeThreads) return;
  reader::dense_merge_row(L.m, blockIdx.x - rows, ws, ws, W, v, out, out, 1);
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
    const auto key_of = [&](int i) { return order_key(x[i]); };
    radix_select(key_of, tokens, remaining, cand, sh, &kth, &need);
    // positions are written after the forced token is merged in, below
    selected = compact_selected(key_of, tokens, kth, need, cand, sh, [&](int i, int, uint32_t) { om[i] = 1; });
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

namespace fl {
// Launch of select_merge_kernel after a dense read of `v` whose partials are at `ws` (W
// waves): the top-k of the read's logits and the merge of its rows into `out`.
int32_t launch_select_merge(const fl_cache_view& v, const float* ws, int W, float* out, const float* logits,
                            int64_t logits_stride, double fraction, int32_t capacity, int32_t* indices,
                            uint8_t* valid, float* mass, float* weights, int32_t* counts, int32_t* nonfinite,
                            hipStream_t st) {
  FL_REQUIRE(select_merge_fits(logits_stride, fraction), "fl_decode_attn_dense_select: logits_stride "
             "above 35840 keys or a selection above 8192 keys (use fl_decode_attn_dense + fl_decode_topk)");
  const TopkArgs A{logits, logits_stride, fraction, capacity, indices, valid, mass, weights, counts, nonfinite};
  const int rows = v.batch * v.heads;
  const int per = static_cast<int>((logits_stride + kTopkThreads - 1) / kTopkThreads);
  const dim3 grid(2 * rows), block(kTopkThreads);
  if (per <= 12)
    hipLaunchKernelGGL(select_merge_kernel<12>, grid, block, 0, st, A, v, ws, W, out);
  else if (per <= 20)
    hipLaunchKernelGGL(select_merge_kernel<20>, grid, block, 0, st, A, v, ws, W, out);
  else
    hipLaunchKernelGGL(select_merge_kernel<kPer>, grid, block, 0, st, A, v, ws, W, out);
  FL_LAUNCH_CHECK("fl_decode_attn_dense_select(select+merge)");
  return FL_OK;
}

bool select_merge_fits(int64_t logits_stride, double fraction) {
  return logits_stride > 0 && logits_stride <= kResKeys &&
         std::ceil(static_cast<double>(logits_stride) * fraction) <= kSelLds;
}
}  // namespace fl

extern "C" int32_t fl_decode_topk(const float* scores, int64_t scores_stride, int32_t rows, const int32_t* n_keys,
                                  int32_t rows_per_count, double fraction, int32_t capacity, int32_t* indices,
                                  uint8_t* valid, float* mass, float* weights, int32_t* counts,
                                  int32_t* nonfinite, void* stream) {
  using namespace fl;
  clear_error();
  FL_REQUIRE(scores && n_keys && indices && valid && mass && weights, "fl_decode_topk: null pointer");
  FL_REQUIRE(rows >= 0 && rows_per_count > 0 && capacity > 0, "fl_decode_topk: bad rows/rows_per_count/capacity");
  FL_REQUIRE(fraction > 0.0 && fraction <= 1.0, "fl_decode_topk: fraction must be in (0, 1]");
  FL_REQUIRE(scores_stride > 0, "fl_decode_topk: bad stride");
  if (rows == 0) return FL_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(rows), block(kTopkThreads);  // block: fallback kernel
  // the stride bounds every row's key count: rows that fit in registers take the one-read kernel
  // keys per thread: the smallest instantiation that holds the row stride
  const int per = static_cast<int>((scores_stride + kTopkThreads - 1) / kTopkThreads);
  if (scores_stride <= kResKeys && std::ceil(static_cast<double>(scores_stride) * fraction) <= kSelLds) {
    if (per <= 12)
      hipLaunchKernelGGL(decode_topk_resident_kernel<12>, grid, block, 0, st, scores, scores_stride, n_keys, rows_per_count,
                       fraction, capacity, indices, valid, mass, weights, counts, nonfinite);
    else if (per <= 20)
      hipLaunchKernelGGL(decode_topk_resident_kernel<20>, grid, block, 0, st, scores, scores_stride, n_keys, rows_per_count,
                       fraction, capacity, indices, valid, mass, weights, counts, nonfinite);
    else
      hipLaunchKernelGGL(decode_topk_resident_kernel<kPer>, grid, block, 0, st, scores, scores_stride, n_keys, rows_per_count,
                       fraction, capacity, indices, valid, mass, weights, counts, nonfinite);
  }
  else
    hipLaunchKernelGGL(decode_topk_kernel, grid, block, 0, st, scores, scores_stride, n_keys, rows_per_count,
                       fraction, capacity, indices, valid, mass, weights, counts, nonfinite);
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
