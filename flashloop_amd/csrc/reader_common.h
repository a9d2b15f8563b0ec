// Helpers shared by the dense and the gather (sparse / selected) decode readers.
#pragma once

#include "fl_common.h"

namespace fl {
namespace reader {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kPartial = kDim + 2;  // m, l, acc[128]



// Byte k of a register to float: these patterns select v_cvt_f32_ubyte{k} (one op).
__device__ __forceinline__ float ubyte0(uint32_t w) { return static_cast<float>(w & 0xFFu); }
__device__ __forceinline__ float ubyte1(uint32_t w) { return static_cast<float>((w >> 8) & 0xFFu); }
__device__ __forceinline__ float ubyte2(uint32_t w) { return static_cast<float>((w >> 16) & 0xFFu); }
__device__ __forceinline__ float ubyte3(uint32_t w) { return static_cast<float>(w >> 24); }

// w & m through v_bitop3_b32 (truth table 0xC0 = S0 & S1).  A plain `&` lets the
// combiner merge the nibble mask with the byte extraction into a bit-field extract,
// which then costs a second instruction per code; bitop3 keeps one mask per word.
__device__ __forceinline__ uint32_t nibble_mask(uint32_t w, uint32_t m) {
  return __builtin_amdgcn_bitop3_b32(w, m, 0u, 0xC0);
}

// 8 nibbles of word w: bytes hold (even channel lo, odd channel hi).
// acc += sum_e qe[e]*lo_e + qo[e]*hi_e, with qo pre-divided by 16 because the high
// nibbles are converted in place (value 16*code).
__device__ __forceinline__ float dot8(uint32_t w, const float* qe, const float* qo, float acc) {
  const uint32_t lo = nibble_mask(w, 0x0F0F0F0Fu);
  const uint32_t hi = nibble_mask(w, 0xF0F0F0F0u);
  acc = fmaf(qe[0], ubyte0(lo), acc);
  acc = fmaf(qe[1], ubyte1(lo), acc);
  acc = fmaf(qe[2], ubyte2(lo), acc);
  acc = fmaf(qe[3], ubyte3(lo), acc);
  acc = fmaf(qo[0], ubyte0(hi), acc);
  acc = fmaf(qo[1], ubyte1(hi), acc);
  acc = fmaf(qo[2], ubyte2(hi), acc);
  acc = fmaf(qo[3], ubyte3(hi), acc);
  return acc;
}

// acc[8 channels of word] += w_even*code (lo) and w_odd16*(16*code) (hi)
__device__ __forceinline__ void axpy8(uint32_t w, float we, float wo, float* acc) {
  const uint32_t lo = nibble_mask(w, 0x0F0F0F0Fu);
  const uint32_t hi = nibble_mask(w, 0xF0F0F0F0u);
  acc[0] = fmaf(we, ubyte0(lo), acc[0]);
  acc[2] = fmaf(we, ubyte1(lo), acc[2]);
  acc[4] = fmaf(we, ubyte2(lo), acc[4]);
  acc[6] = fmaf(we, ubyte3(lo), acc[6]);
  acc[1] = fmaf(wo, ubyte0(hi), acc[1]);
  acc[3] = fmaf(wo, ubyte1(hi), acc[3]);
  acc[5] = fmaf(wo, ubyte2(hi), acc[5]);
  acc[7] = fmaf(wo, ubyte3(hi), acc[7]);
}

// Codes read as fp16 subnormals: masking a word with 0x000F000F (0x00F000F0) leaves in
// each 16-bit half one nibble c (16c) below bit 10, the fp16 value c*2^-24 (16c*2^-24),
// which v_fma_mix_f32 and v_dot2_f32_f16 take as exact operands.  Two masks per four
// codes replace four conversions; the factors carry the 2^24 (and the odd channels' 1/16).
__device__ __forceinline__ float h16lo(uint32_t x) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(x & 0xFFFFu)));
}
__device__ __forceinline__ float h16hi(uint32_t x) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(x >> 16)));
}
// acc[c] += we*code_c for even channels, wo*(16*code_c) for odd ones (we, wo scaled by 2^24)
__device__ __forceinline__ void axpy8h(uint32_t w, float we, float wo, float* acc) {
  const uint32_t x0 = w & 0x000F000Fu, x1 = w & 0x00F000F0u;
  const uint32_t w8 = w >> 8;
  const uint32_t x2 = w8 & 0x000F000Fu, x3 = w8 & 0x00F000F0u;
  acc[0] = fmaf(we, h16lo(x0), acc[0]);
  acc[4] = fmaf(we, h16hi(x0), acc[4]);
  acc[1] = fmaf(wo, h16lo(x1), acc[1]);
  acc[5] = fmaf(wo, h16hi(x1), acc[5]);
  acc[2] = fmaf(we, h16lo(x2), acc[2]);
  acc[6] = fmaf(we, h16hi(x2), acc[6]);
  acc[3] = fmaf(wo, h16lo(x3), acc[3]);
  acc[7] = fmaf(wo, h16hi(x3), acc[7]);
}
constexpr float kSub16 = 16777216.0f;  // 2^24: fp16 subnormal code c reads as c * 2^-24

// The K contraction of one code word against fp16 factor pairs, two channels per
// v_dot2_f32_f16: f.x = (f0, f4), f.y = (f1, f5)/16, f.z = (f2, f6), f.w = (f3, f7)/16
// for channels 0..7 of the word, whose masked codes are fp16 subnormals c*2^-24 (16c*2^-24
// for the odd ones).  The products are exact in fp32; the result carries 2^-24.
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float dot8h2(uint32_t w, uint4 f, float acc) {
  const uint32_t w8 = w >> 8;
  acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, w & 0x000F000Fu), __builtin_bit_cast(half2_t, f.x), acc, false);
  acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, w & 0x00F000F0u), __builtin_bit_cast(half2_t, f.y), acc, false);
  acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, w8 & 0x000F000Fu), __builtin_bit_cast(half2_t, f.z), acc, false);
  acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, w8 & 0x00F000F0u), __builtin_bit_cast(half2_t, f.w), acc, false);
  return acc;
}
// Position (in fp16 units) of channel c's factor in the pair layout dot8h2 reads: word
// c/8 holds 8 factors, pair (c%8)%4, half (c%8)/4.
__device__ __forceinline__ int pair_slot(int c) { return (c >> 3) * 8 + (c & 3) * 2 + ((c >> 2) & 1); }

struct QuadState {
  float m, l, mu;
  float acc[32];
};

// Branch-free (selects, no early exit): a divergent exit here joins the caller's control
// flow, and at that join the compiler waits for every load in flight, including the next
// rows already requested.
__device__ __forceinline__ void online_update(QuadState& st, const float* lg, float* p, int n) {
  float mloc = st.m;
  for (int i = 0; i < n; ++i) mloc = fmaxf(mloc, lg[i]);
  const bool none = mloc == -INFINITY;  // nothing valid yet: state unchanged, p = 0
  const float alpha = none ? 1.0f : fast_exp2((st.m - mloc) * kLog2e);
  float ps = 0.0f;
  for (int i = 0; i < n; ++i) {
    p[i] = none ? 0.0f : fast_exp2((lg[i] - mloc) * kLog2e);
    ps += p[i];
  }
  st.l = st.l * alpha + ps;
  st.mu *= alpha;
#pragma unroll
  for (int c = 0; c < 32; ++c) st.acc[c] *= alpha;
  st.m = mloc;
}

// Merge the 64 quad states of the workgroup and write one partial (m, l, acc[128]).
__device__ void write_partial(QuadState& st, float* part, float (*comb)[16][kDim], float* lsh, float* msh) {
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, quarter = lane & 3, row = lane >> 2;
  const float mw = wave_max(st.m);
  if (lane == 0) msh[wave] = mw;
  __syncthreads();
  float M = msh[0];
  for (int w = 1; w < kWaves; ++w) M = fmaxf(M, msh[w]);
  const float f = (st.m == -INFINITY) ? 0.0f : fast_exp2((st.m - M) * kLog2e);
#pragma unroll
  for (int c = 0; c < 32; ++c) comb[wave][row][32 * quarter + c] = (st.acc[c] + st.mu) * f;
  if (quarter == 0) lsh[wave * 16 + row] = st.l * f;
  __syncthreads();
  if (tid < kDim) {
    float s = 0.0f;
    for (int w = 0; w < kWaves; ++w)
      for (int r = 0; r < 16; ++r) s += comb[w][r][tid];
    part[2 + tid] = s;
  } else if (tid == kDim) {
    float s = 0.0f;
    for (int i = 0; i < kWaves * 16; ++i) s += lsh[i];
    part[0] = M;
    part[1] = s;
  }
}

enum MergeMode { kMergeSoftmax = 0, kMergeMassDelta = 1, kMergeSum = 2 };

// Combine a row's partials (m, l, acc[128]).
//   kMergeSoftmax:   out = sum_i e^{m_i-M} acc_i / sum_i e^{m_i-M} l_i
//   kMergeMassDelta: out = mass * (softmax merge - src)
//   kMergeSum:       out = sum_i acc_i
//   kMergeMassDeltaFused: src = sum_i acc2_i (second partial set, written to src_out),
//                    out = mass * (softmax merge - src)
// Latency-bound, so every stage issues its loads at once: the per-part weights e^{m_i-M}
// are formed by all threads into LDS, and each channel's sum is split over kMergeSplit
// thread groups whose partial sums meet in LDS.
constexpr int kMergeMassDeltaFused = 3;
constexpr int kMergeMaxParts = 4096;
constexpr int kMergeSplit = 4;
constexpr int kMergeThreads = kDim * kMergeSplit;

// Part i of the row: `base + i*kPartial` for i < n_main, `extra` for i == n_main.
struct MergeParts {
  const float* base;
  int n_main;
  const float* extra;  // optional extra part (nullptr: none)
  __device__ __forceinline__ int count() const { return n_main + (extra ? 1 : 0); }
  __device__ __forceinline__ const float* part(int i) const {
    return i < n_main ? base + static_cast<int64_t>(i) * kPartial : extra;
  }
};

struct MergeLdsBuf {
  float f[kMergeMaxParts];
  float red[kMergeThreads / kWave];
  float acc[kMergeSplit][kDim];
};

// Softmax merge of one row into out[c] (thread c < kDim writes); returns nothing.
__device__ __forceinline__ float block_max_merge(float x, float* red) {
  const int tid = threadIdx.x;
  x = wave_max(x);
  if ((tid & 63) == 0) red[tid >> 6] = x;
  __syncthreads();
  float r = red[0];
  for (int w = 1; w < kMergeThreads / kWave; ++w) r = fmaxf(r, red[w]);
  __syncthreads();
  return r;
}
__device__ __forceinline__ float block_sum_merge(float x, float* red) {
  const int tid = threadIdx.x;
  x = wave_sum(x);
  if ((tid & 63) == 0) red[tid >> 6] = x;
  __syncthreads();
  float r = 0.0f;
  for (int w = 0; w < kMergeThreads / kWave; ++w) r += red[w];
  __syncthreads();
  return r;
}

// Channel sums sum_i w_i * part_i[2 + c] (w from LDS, or 1), split over kMergeSplit groups.
template <bool WEIGHTED>
__device__ __forceinline__ float merge_channel_sum(const MergeParts& P, const float* f, float (*acc)[kDim]) {
  const int tid = threadIdx.x, c = tid & (kDim - 1), j = tid / kDim;
  const int n = min(P.count(), kMergeMaxParts);
  float s = 0.0f;
#pragma unroll 16
  for (int i = j; i < n; i += kMergeSplit) {
    const float x = P.part(i)[2 + c];
    s = WEIGHTED ? fmaf(x, f[i], s) : s + x;
  }
  acc[j][c] = s;
  __syncthreads();
  float r = 0.0f;
  if (tid < kDim)
#pragma unroll
    for (int k = 0; k < kMergeSplit; ++k) r += acc[k][tid];
  __syncthreads();
  return r;  // valid for tid < kDim
}

__device__ __forceinline__ float merge_softmax_general(const MergeParts& P, MergeLdsBuf& S) {
  const int tid = threadIdx.x;
  const int n = min(P.count(), kMergeMaxParts);
  // (m, l) of this thread's parts are loaded once, in one round, and kept in registers
  constexpr int kPer = kMergeMaxParts / kMergeThreads;
  float mi[kPer], li[kPer];
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int i = tid + k * kMergeThreads;
    mi[k] = -INFINITY;
    li[k] = 0.0f;
    if (i < n) {
      const float* p = P.part(i);
      mi[k] = p[0];
      li[k] = p[1];
    }
  }
  float M = -INFINITY;
#pragma unroll
  for (int k = 0; k < kPer; ++k) M = fmaxf(M, mi[k]);
  M = block_max_merge(M, S.red);
  float L = 0.0f;
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int i = tid + k * kMergeThreads;
    if (i < n) {
      const float fi = (mi[k] == -INFINITY) ? 0.0f : fast_exp2((mi[k] - M) * kLog2e);
      S.f[i] = fi;
      L = fmaf(li[k], fi, L);
    }
  }
  L = block_sum_merge(L, S.red);  // also orders the f[] writes before the reads below
  const float acc = merge_channel_sum<true>(P, S.f, S.acc);
  return acc / L;
}

// Softmax merge with every load in one round: thread (c, j) loads m, l and channel c of
// parts j, j+kMergeSplit, ... (up to kMergeLocal each) before any arithmetic.
constexpr int kMergeLocal = 8;

__device__ __forceinline__ float merge_softmax(const MergeParts& P, MergeLdsBuf& S) {
  const int n = min(P.count(), kMergeMaxParts);
  if (n > kMergeSplit * kMergeLocal) return merge_softmax_general(P, S);
  const int tid = threadIdx.x, c = tid & (kDim - 1), j = tid / kDim;
  float mi[kMergeLocal], li[kMergeLocal], ai[kMergeLocal];
#pragma unroll
  for (int k = 0; k < kMergeLocal; ++k) {
    const int i = j + kMergeSplit * k;
    mi[k] = -INFINITY;
    li[k] = 0.0f;
    ai[k] = 0.0f;
    if (i < n) {
      const float* p = P.part(i);
      mi[k] = p[0];
      li[k] = p[1];
      ai[k] = p[2 + c];
    }
  }
  float M = mi[0];
#pragma unroll
  for (int k = 1; k < kMergeLocal; ++k) M = fmaxf(M, mi[k]);
  M = block_max_merge(M, S.red);
  float L = 0.0f, acc = 0.0f;
#pragma unroll
  for (int k = 0; k < kMergeLocal; ++k) {
    const float e = (mi[k] == -INFINITY) ? 0.0f : fast_exp2((mi[k] - M) * kLog2e);
    L = fmaf(li[k], e, L);
    acc = fmaf(ai[k], e, acc);
  }
  // L: every part counted once (by the c == 0 thread of its split group)
  L = block_sum_merge(c == 0 ? L : 0.0f, S.red);
  S.acc[j][c] = acc;
  __syncthreads();
  float r = 0.0f;
  if (tid < kDim)
#pragma unroll
    for (int k = 0; k < kMergeSplit; ++k) r += S.acc[k][tid];
  return r / L;  // valid for tid < kDim
}

__global__ __launch_bounds__(kMergeThreads) void merge_partials_kernel(const float* ws, int nparts, float* out,
                                                                       int mode, const float* mass, const float* src,
                                                                       const float* ws2, float* src_out) {
  __shared__ MergeLdsBuf S;
  const int bh = blockIdx.x, tid = threadIdx.x;
  const int64_t o = static_cast<int64_t>(bh) * kDim + tid;
  const MergeParts P{ws + static_cast<int64_t>(bh) * nparts * kPartial, nparts, nullptr};
  if (mode == kMergeSum) {
    const float r = merge_channel_sum<false>(P, nullptr, S.acc);
    if (tid < kDim) out[o] = r;
    return;
  }
  float res = merge_softmax(P, S);
  if (mode == kMergeMassDeltaFused) {
    const MergeParts P2{ws2 + static_cast<int64_t>(bh) * nparts * kPartial, nparts, nullptr};
    const float s = merge_channel_sum<false>(P2, nullptr, S.acc);
    if (tid < kDim) {
      src_out[o] = s;
      res = mass[bh] * (res - s);
    }
  } else if (mode == kMergeMassDelta) {
    if (tid < kDim) res = mass[bh] * (res - src[o]);
  }
  if (tid < kDim) out[o] = res;
}

}  // namespace
}  // namespace reader
}  // namespace fl
