// J1: int4 quantize-and-pack of 64-token temporal groups through the cross-loop
// residual chain (flashloop_torch/kv_quantization.py:395-414, 531-650).
//
// One workgroup (256 threads) encodes one group of one (batch, head) for all loops,
// either its K chain (blockIdx.z == 0) or its V chain (blockIdx.z == 1): K (per channel
// over 64 tokens) and V (per token over 64-channel halves) are independent chains.  Each
// thread keeps the elements it owns in registers across loops; the nibble transposition
// of K goes through wave-private LDS.
//
// Bit-exactness: every float op is a single IEEE op with explicit rounding
// (__fsub_rn/__fmul_rn/__fadd_rn/__fmaf_rn, no contraction), rintf is round-half-even,
// and bf16 narrowing is round-to-nearest-even -- the values of the reference's eager
// torch-CPU codec.  Its division is computed as an exact Markstein quotient (encode).
#include "fl_common.h"

#include <type_traits>

namespace fl {
namespace {

struct PackArgs {
  fl_cache_view v;
  int loops;
  const uint16_t* src_k[4];
  const uint16_t* src_v[4];
  int64_t src_bh_stride;
  int src_row_offset;
  const uint8_t* mask[2];
  int64_t mask_stride;
  const int32_t* dst_group0;
  uint16_t* rk[4];
  uint16_t* rv[4];
};

struct Quant {
  float scale, minimum, inv;  // inv = RN(1/scale)
};

__device__ __forceinline__ Quant make_quant(float mn, float mx, bool any) {
  if (!any) {
    mn = 0.0f;
    mx = 0.0f;
  }
  // A group whose smallest value is a zero keeps +0 as its minimum (-0 + +0 = +0):
  // which zero a min reduction returns over a mix of +0 and -0 depends on its
  // evaluation order.  Reconstructions are the same either way.
  mn = __fadd_rn(mn, 0.0f);
  const float span = __fsub_rn(mx, mn);
  const float scale = span > 0.0f ? __fdiv_rn(span, 15.0f) : 1.0f;
  return {scale, mn, __fdiv_rn(1.0f, scale)};
}

// bf16 narrowing (round to nearest even) and back, on the hardware conversion
// (v_cvt_pk_bf16_f32): the same value as round_bf16 for every non-NaN input (checked
// on the device over all 2^32 float patterns).
// Two values per conversion instruction.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void round_bf16_pair(float& a, float& b) {
  const f32x2_t f = {a, b};
  const uint32_t w = __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_t));
  a = __uint_as_float(w << 16);
  b = __uint_as_float(w & 0xFFFF0000u);
}

// Two values that are already bf16 (their low 16 bits zero, as every reconstruction
// here is after round_bf16_pair) as one packed bf16 pair: their upper halves.
__device__ __forceinline__ uint32_t bf16_bits_pair(float lo, float hi) {
  return (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xFFFF0000u);
}

// code = clamp(rint((x - minimum) / scale), 0, 15).  The quotient is Markstein's
// correction of a * RN(1/scale): with y = RN(1/b), q0 = RN(a*y) and the exact remainder
// r = a - b*q0 (one fma), RN(q0 + r*y) is the correctly rounded a/b (P. Markstein,
// IBM J. Res. Dev. 34(1), 1990).  Three ops instead of an IEEE division per element.
// The remainder is exact only while b*q0 stays clear of the subnormal range, which holds
// for scale >= kMinFastScale over every quotient that can round to a nonzero code; groups
// whose span is smaller than that (scale subnormal or near it, where 1/scale can even
// overflow) take the IEEE division instead (exact_div).  tests/markstein_check.c checks
// both against the division over the codec's domain, subnormal spans included.
constexpr float kMinFastScale = 0x1p-100f;

__device__ __forceinline__ bool needs_exact_div(Quant q) { return !(q.scale >= kMinFastScale); }

// Returns the code as a float (an integer in [0, 15]): the decode takes it as it is,
// with no conversion back from the integer.
template <bool EXACT_DIV>
__device__ __forceinline__ float encode(float x, Quant q) {
  const float a = __fsub_rn(x, q.minimum);
  float c;
  if constexpr (EXACT_DIV) {
    c = rintf(__fdiv_rn(a, q.scale));
  } else {
    const float q0 = __fmul_rn(a, q.inv);
    const float r = __fmaf_rn(-q0, q.scale, a);
    c = rintf(__fmaf_rn(r, q.inv, q0));
  }
  return fminf(fmaxf(c, 0.0f), 15.0f);
}

// code * scale + minimum before its bf16 rounding (round_bf16_pair)
__device__ __forceinline__ float decode_f32(float code, Quant q) {
  return __fadd_rn(__fmul_rn(code, q.scale), q.minimum);
}

// Raw buffer over `bytes` bytes at p (wave-uniform).  Loads past the end, or from a
// null p with zero bytes, return zero without touching memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t pack_res(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, static_cast<int>(bytes), 0x00020000);
}

// Per-token inputs of one loop, loaded ahead of their use: the loop's mask byte and the
// token's rank-map entry (loops 3/4).  Loops 1/2 keep every token at its own row.
struct TokenIn {
  uint32_t mask;
  int rank;
};

template <int R>
__device__ __forceinline__ TokenIn token_load(const PackArgs& a, int b, int g, int src_row0, int i) {
  if constexpr (R < 2) {
    return {1u, g * kGroup + i};
  } else {
    const uint8_t* m = a.mask[R - 2];
    const auto mr = pack_res(m ? m + static_cast<int64_t>(b) * a.mask_stride : nullptr,
                             m ? static_cast<uint32_t>(a.mask_stride) : 0u);
    const uint32_t byte = __builtin_amdgcn_raw_buffer_load_b8(mr, src_row0 + i, 0, 0);
    const int rank = a.v.rank[R - 2][static_cast<int64_t>(b) * a.v.token_capacity + g * kGroup + i];
    return {byte, rank};
  }
}

// Token active in loop R (kv_quantization.py:465: loops 3/4 follow their masks; no mask
// means every token).
template <int R>
__device__ __forceinline__ bool token_active(const PackArgs& a, TokenIn t) {
  if constexpr (R < 2) return true;
  else return a.mask[R - 2] == nullptr || t.mask != 0;
}

// Destination row of the token in stream R (-1: not stored).
template <int R>
__device__ __forceinline__ int token_row(const PackArgs& a, TokenIn t) {
  if constexpr (R < 2) return t.rank;
  else return token_active<R>(a, t) && t.rank < a.v.row_capacity[R] ? t.rank : -1;
}

// ---------------------------------------------------------------------------------
// K chain (workgroups with blockIdx.z == 0).  Thread (pair = tid/4, quarter = tid%4) owns
// channels 2*pair, 2*pair+1 of tokens 16*quarter .. +16, so wave w holds channels
// 32w .. 32w+31 of all 64 tokens: the 16-byte chunk w of every code row.  The nibble
// transposition therefore stays inside the wave (wave-private LDS, no workgroup barrier),
// and lane i then stores row i's chunk.  Loop r+1's source words and token inputs are
// requested before loop r computes.
// ---------------------------------------------------------------------------------
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int R>
__device__ __forceinline__ void load_k_words(uint32_t (&w)[16], const PackArgs& a, int64_t src_base, int pair,
                                             int quarter) {
#pragma unroll
  for (int k = 0; k < 16; ++k)
    w[k] = *reinterpret_cast<const uint32_t*>(a.src_k[R] + src_base + static_cast<int64_t>(quarter * 16 + k) * kDim +
                                              2 * pair);
}

template <int R, int LOOPS>
__device__ __forceinline__ void key_loop(const PackArgs& a, int b, int bh, int g, int src_row0, int64_t src_base,
                                         uint32_t (&w)[16], uint32_t (&w_next)[16], TokenIn tin, TokenIn& tin_next,
                                         float (&r0)[16], float (&r1)[16], uint8_t (*lds)[16]) {
  const fl_cache_view& v = a.v;
  const int tid = threadIdx.x, lane = tid & 63, pair = tid >> 2, quarter = tid & 3;
  if constexpr (R + 1 < LOOPS) {
    load_k_words<R + 1>(w_next, a, src_base, pair, quarter);
    tin_next = token_load<R + 1>(a, b, g, src_row0, lane);
  }
  // active tokens of this loop, one bit per token (lane i holds token i); loops 1/2
  // have every token of a packed group (a constant, so the per-element tests fold away)
  const uint64_t act = R < 2 ? ~0ull : __ballot(token_active<R>(a, tin));
  float x0[16], x1[16];
  float mn0 = INFINITY, mx0 = -INFINITY, mn1 = INFINITY, mx1 = -INFINITY;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const float l0 = bf16lo_to_f32(w[k]), l1 = bf16hi_to_f32(w[k]);
    if constexpr (R == 0) {
      x0[k] = l0;
      x1[k] = l1;
    } else {
      x0[k] = __fsub_rn(l0, r0[k]);
      x1[k] = __fsub_rn(l1, r1[k]);
      round_bf16_pair(x0[k], x1[k]);
    }
    if ((act >> (quarter * 16 + k)) & 1) {
      mn0 = fminf(mn0, x0[k]);
      mx0 = fmaxf(mx0, x0[k]);
      mn1 = fminf(mn1, x1[k]);
      mx1 = fmaxf(mx1, x1[k]);
    }
  }
  mn0 = quad_min(mn0);
  mx0 = quad_max(mx0);
  mn1 = quad_min(mn1);
  mx1 = quad_max(mx1);
  const Quant q0 = make_quant(mn0, mx0, act != 0);
  const Quant q1 = make_quant(mn1, mx1, act != 0);
  if (quarter == 0) {
    const float4 meta = make_float4(q0.scale, q0.minimum, q1.scale, q1.minimum);
    const int64_t mi = ((static_cast<int64_t>(bh) * (v.token_capacity / kGroup) + g) * kDim + 2 * pair) * 2;
    *reinterpret_cast<float4*>(v.key_meta[R] + mi) = meta;
    const uint2 half_meta = make_uint2(
        static_cast<uint32_t>(f32_to_f16(q0.scale)) | (static_cast<uint32_t>(f32_to_f16(q0.minimum)) << 16),
        static_cast<uint32_t>(f32_to_f16(q1.scale)) | (static_cast<uint32_t>(f32_to_f16(q1.minimum)) << 16));
    *reinterpret_cast<uint2*>(v.key_meta_half[R] + mi) = half_meta;
  }
  // The encode loop is instantiated twice; a wave takes the IEEE-division form only when
  // one of its groups has a scale below kMinFastScale (a wave-uniform branch).
  auto encode_rows = [&](auto exact) __attribute__((always_inline)) {
    constexpr bool EXACT = decltype(exact)::value;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int i = quarter * 16 + k;
      uint32_t c0 = 0, c1 = 0;
      float d0 = 0.0f, d1 = 0.0f;
      if ((act >> i) & 1) {
        const float f0 = encode<EXACT>(x0[k], q0), f1 = encode<EXACT>(x1[k], q1);
        c0 = static_cast<uint32_t>(f0);
        c1 = static_cast<uint32_t>(f1);
        d0 = decode_f32(f0, q0);
        d1 = decode_f32(f1, q1);
        round_bf16_pair(d0, d1);
      }
      lds[i][pair & 15] = static_cast<uint8_t>(c0 | (c1 << 4));
      if constexpr (R == 0) {
        r0[k] = d0;
        r1[k] = d1;
      } else {
        // inactive rows add an exact zero delta (kv_quantization.py:465)
        r0[k] = __fadd_rn(r0[k], d0);
        r1[k] = __fadd_rn(r1[k], d1);
        round_bf16_pair(r0[k], r1[k]);
      }
    }
  };
  if (__builtin_expect(__any(needs_exact_div(q0) || needs_exact_div(q1)), 0)) encode_rows(std::true_type{});
  else encode_rows(std::false_type{});
  // audit copy of the reconstruction (one branch, outside the encode loop)
  if (a.rk[R] != nullptr) {
#pragma unroll
    for (int k = 0; k < 16; ++k)
      *reinterpret_cast<uint32_t*>(a.rk[R] + src_base + static_cast<int64_t>(quarter * 16 + k) * kDim + 2 * pair) =
          bf16_bits_pair(r0[k], r1[k]);
  }
  wave_lds_sync();
  const int row = token_row<R>(a, tin);
  const uint4 chunk = *reinterpret_cast<const uint4*>(lds[lane]);
  if (row >= 0)
    *reinterpret_cast<uint4*>(v.key_codes[R] + (static_cast<int64_t>(bh) * v.row_capacity[R] + row) * kCodeStride +
                              (tid >> 6) * 16) = chunk;
  wave_lds_sync();  // the chunk reads are done before the next loop's writes
}

template <int LOOPS>
__device__ __forceinline__ void pack_keys(const PackArgs& a, int b, int bh, int g, int src_row0, int64_t src_base) {
  __shared__ uint8_t lds[kDim / 32][kGroup][16];
  const int tid = threadIdx.x, lane = tid & 63;
  uint32_t wa[16], wb[16];
  TokenIn ta = token_load<0>(a, b, g, src_row0, lane), tb{};
  load_k_words<0>(wa, a, src_base, tid >> 2, tid & 3);
  float r0[16], r1[16];
  uint8_t(*mine)[16] = lds[tid >> 6];
  key_loop<0, LOOPS>(a, b, bh, g, src_row0, src_base, wa, wb, ta, tb, r0, r1, mine);
  if constexpr (LOOPS > 1) key_loop<1, LOOPS>(a, b, bh, g, src_row0, src_base, wb, wa, tb, ta, r0, r1, mine);
  if constexpr (LOOPS > 2) key_loop<2, LOOPS>(a, b, bh, g, src_row0, src_base, wa, wb, ta, tb, r0, r1, mine);
  if constexpr (LOOPS > 3) key_loop<3, LOOPS>(a, b, bh, g, src_row0, src_base, wb, wa, tb, ta, r0, r1, mine);
}

// ---------------------------------------------------------------------------------
// V chain (workgroups with blockIdx.z == 1).  Thread (i = tid/4, quarter = tid%4) owns
// channels 32*quarter .. +32 of token i (V groups are 64-channel halves, quarter/2).
// Loop r+1's source row and token inputs are requested before loop r computes.
// ---------------------------------------------------------------------------------
template <int R>
__device__ __forceinline__ void load_v_words(uint4 (&w)[4], const PackArgs& a, int64_t row_off) {
  const uint4* src = reinterpret_cast<const uint4*>(a.src_v[R] + row_off);
#pragma unroll
  for (int k = 0; k < 4; ++k) w[k] = src[k];
}

template <int R, int LOOPS>
__device__ __forceinline__ void value_loop(const PackArgs& a, int b, int bh, int g, int src_row0, int64_t row_off,
                                           uint4 (&w)[4], uint4 (&w_next)[4], TokenIn tin, TokenIn& tin_next,
                                           float (&rv)[32]) {
  const fl_cache_view& v = a.v;
  const int i = threadIdx.x >> 2, quarter = threadIdx.x & 3, half = quarter >> 1;
  if constexpr (R + 1 < LOOPS) {
    load_v_words<R + 1>(w_next, a, row_off);
    tin_next = token_load<R + 1>(a, b, g, src_row0, i);
  }
  const bool act = token_active<R>(a, tin);
  float x[32];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t ws[4] = {w[k].x, w[k].y, w[k].z, w[k].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[8 * k + 2 * e] = bf16lo_to_f32(ws[e]);
      x[8 * k + 2 * e + 1] = bf16hi_to_f32(ws[e]);
    }
  }
  if constexpr (R > 0) {
#pragma unroll
    for (int c = 0; c < 32; c += 2) {
      x[c] = __fsub_rn(x[c], rv[c]);
      x[c + 1] = __fsub_rn(x[c + 1], rv[c + 1]);
      round_bf16_pair(x[c], x[c + 1]);
    }
  }
  float mn = INFINITY, mx = -INFINITY;
#pragma unroll
  for (int c = 0; c < 32; ++c) {
    mn = fminf(mn, x[c]);
    mx = fmaxf(mx, x[c]);
  }
  mn = pair_min(mn);
  mx = pair_max(mx);
  const Quant q = make_quant(mn, mx, act);
  uint32_t words[4] = {0, 0, 0, 0};
  auto encode_row = [&](auto exact) __attribute__((always_inline)) {
    constexpr bool EXACT = decltype(exact)::value;
#pragma unroll
    for (int c = 0; c < 32; c += 2) {
      uint32_t c0 = 0, c1 = 0;
      float d0 = 0.0f, d1 = 0.0f;
      if (act) {
        const float f0 = encode<EXACT>(x[c], q), f1 = encode<EXACT>(x[c + 1], q);
        c0 = static_cast<uint32_t>(f0);
        c1 = static_cast<uint32_t>(f1);
        d0 = decode_f32(f0, q);
        d1 = decode_f32(f1, q);
        round_bf16_pair(d0, d1);
      }
      words[c >> 3] |= (c0 | (c1 << 4)) << (4 * (c & 7));
      if constexpr (R == 0) {
        rv[c] = d0;
        rv[c + 1] = d1;
      } else {
        rv[c] = __fadd_rn(rv[c], d0);
        rv[c + 1] = __fadd_rn(rv[c + 1], d1);
        round_bf16_pair(rv[c], rv[c + 1]);
      }
    }
  };
  if (__builtin_expect(__any(needs_exact_div(q)), 0)) encode_row(std::true_type{});
  else encode_row(std::false_type{});
  const int row = token_row<R>(a, tin);
  if (row >= 0) {
    const int t = g * kGroup + i;
    const int64_t rowi = static_cast<int64_t>(bh) * v.row_capacity[R] + row;
    *reinterpret_cast<uint4*>(v.value_codes[R] + rowi * kCodeStride + 16 * quarter) =
        make_uint4(words[0], words[1], words[2], words[3]);
    if ((quarter & 1) == 0) {
      *reinterpret_cast<float2*>(v.value_meta[R] + (rowi * 2 + half) * 2) = make_float2(q.scale, q.minimum);
      *reinterpret_cast<uint32_t*>(v.value_meta_half[R] + (rowi * 2 + half) * 2) =
          static_cast<uint32_t>(f32_to_f16(q.scale)) | (static_cast<uint32_t>(f32_to_f16(q.minimum)) << 16);
      const int64_t rec = ((static_cast<int64_t>(bh) * v.token_capacity + t) * 2 + half) * 4 + R;
      *reinterpret_cast<float2*>(v.value_meta_token + rec * 2) = make_float2(q.scale, q.minimum);
    }
  }
  if (a.rv[R] != nullptr) {
    uint4* dst = reinterpret_cast<uint4*>(a.rv[R] + row_off);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint32_t o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        o[e] = bf16_bits_pair(rv[8 * k + 2 * e], rv[8 * k + 2 * e + 1]);
      }
      dst[k] = make_uint4(o[0], o[1], o[2], o[3]);
    }
  }
}

template <int LOOPS>
__device__ __forceinline__ void pack_values(const PackArgs& a, int b, int bh, int g, int src_row0, int64_t src_base) {
  const int i = threadIdx.x >> 2, quarter = threadIdx.x & 3;
  const int64_t row_off = src_base + static_cast<int64_t>(i) * kDim + 32 * quarter;
  uint4 wa[4], wb[4];
  TokenIn ta = token_load<0>(a, b, g, src_row0, i), tb{};
  load_v_words<0>(wa, a, row_off);
  float rv[32];
  value_loop<0, LOOPS>(a, b, bh, g, src_row0, row_off, wa, wb, ta, tb, rv);
  if constexpr (LOOPS > 1) value_loop<1, LOOPS>(a, b, bh, g, src_row0, row_off, wb, wa, tb, ta, rv);
  if constexpr (LOOPS > 2) value_loop<2, LOOPS>(a, b, bh, g, src_row0, row_off, wa, wb, ta, tb, rv);
  if constexpr (LOOPS > 3) value_loop<3, LOOPS>(a, b, bh, g, src_row0, row_off, wb, wa, tb, ta, rv);
}

// One workgroup per (group j, row bh, chain z): z = 0 encodes the group's K chain over all
// loops, z = 1 its V chain (the chains are independent).
template <int LOOPS>
__global__ __launch_bounds__(256) void pack_groups_kernel(PackArgs a) {
  const fl_cache_view& v = a.v;
  const int j = blockIdx.x;
  const int bh = blockIdx.y;
  const int b = bh / v.heads;
  const int g0 = a.dst_group0[b];
  if (g0 < 0) return;
  const int g = g0 + j;
  if ((g + 1) * kGroup > v.token_capacity) return;  // outside the destination
  const int src_row0 = a.src_row_offset + j * kGroup;
  const int64_t src_base = (static_cast<int64_t>(bh) * a.src_bh_stride + src_row0) * kDim;
  if (blockIdx.z == 0) pack_keys<LOOPS>(a, b, bh, g, src_row0, src_base);
  else pack_values<LOOPS>(a, b, bh, g, src_row0, src_base);
}

}  // namespace
}  // namespace fl

extern "C" int32_t fl_pack_kv_groups(const fl_cache_view* view, int32_t loops,
                                     const uint16_t* const* src_keys, const uint16_t* const* src_values,
                                     int64_t src_bh_stride, int32_t src_row_offset,
                                     const uint8_t* const* masks, int64_t mask_stride,
                                     const int32_t* dst_group0, int32_t n_groups,
                                     uint16_t* const* recon_keys, uint16_t* const* recon_values,
                                     void* stream) {
  using namespace fl;
  clear_error();
  FL_REQUIRE(view != nullptr, "fl_pack_kv_groups: view is null");
  const fl_cache_view& v = *view;
  FL_REQUIRE(loops >= 1 && loops <= 4, "fl_pack_kv_groups: loops must be in 1..4");
  FL_REQUIRE(v.batch > 0 && v.heads > 0, "fl_pack_kv_groups: empty batch/heads");
  FL_REQUIRE(v.token_capacity > 0 && v.token_capacity % kGroup == 0,
             "fl_pack_kv_groups: token_capacity must be a positive multiple of 64");
  FL_REQUIRE(src_keys != nullptr && src_values != nullptr && dst_group0 != nullptr,
             "fl_pack_kv_groups: null sources or dst_group0");
  FL_REQUIRE(n_groups >= 0, "fl_pack_kv_groups: negative n_groups");
  FL_REQUIRE(src_row_offset >= 0 && src_bh_stride >= static_cast<int64_t>(src_row_offset) + 64LL * n_groups,
             "fl_pack_kv_groups: source rows exceed src_bh_stride");
  PackArgs a{};
  a.v = v;
  a.loops = loops;
  for (int r = 0; r < loops; ++r) {
    FL_REQUIRE(src_keys[r] && src_values[r], "fl_pack_kv_groups: null source for a loop");
    FL_REQUIRE(v.key_codes[r] && v.key_meta[r] && v.value_codes[r] && v.value_meta[r] && v.value_meta_token &&
                   v.key_meta_half[r] && v.value_meta_half[r],
               "fl_pack_kv_groups: destination stream pointer is null");
    FL_REQUIRE(reinterpret_cast<uintptr_t>(src_keys[r]) % 16 == 0 && reinterpret_cast<uintptr_t>(src_values[r]) % 16 == 0,
               "fl_pack_kv_groups: sources must be 16-byte aligned");
    a.src_k[r] = src_keys[r];
    a.src_v[r] = src_values[r];
    a.rk[r] = recon_keys ? recon_keys[r] : nullptr;
    a.rv[r] = recon_values ? recon_values[r] : nullptr;
    if (r >= 2) {
      FL_REQUIRE(v.rank[r - 2] != nullptr, "fl_pack_kv_groups: loops 3/4 need rank maps");
      FL_REQUIRE(v.row_capacity[r] >= 0, "fl_pack_kv_groups: negative row capacity");
    } else {
      FL_REQUIRE(v.row_capacity[r] == v.token_capacity, "fl_pack_kv_groups: streams 0/1 rows must equal token_capacity");
    }
  }
  a.src_bh_stride = src_bh_stride;
  a.src_row_offset = src_row_offset;
  a.mask[0] = masks ? masks[0] : nullptr;
  a.mask[1] = masks ? masks[1] : nullptr;
  FL_REQUIRE((a.mask[0] == nullptr && a.mask[1] == nullptr) || mask_stride >= static_cast<int64_t>(src_row_offset) + 64LL * n_groups,
             "fl_pack_kv_groups: mask_stride too small");
  a.mask_stride = mask_stride;
  a.dst_group0 = dst_group0;
  if (n_groups == 0) return FL_OK;
  const dim3 grid(n_groups, v.batch * v.heads, 2);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  switch (loops) {
    case 1: hipLaunchKernelGGL(pack_groups_kernel<1>, grid, dim3(256), 0, st, a); break;
    case 2: hipLaunchKernelGGL(pack_groups_kernel<2>, grid, dim3(256), 0, st, a); break;
    case 3: hipLaunchKernelGGL(pack_groups_kernel<3>, grid, dim3(256), 0, st, a); break;
    default: hipLaunchKernelGGL(pack_groups_kernel<4>, grid, dim3(256), 0, st, a); break;
  }
  FL_LAUNCH_CHECK("fl_pack_kv_groups");
  return FL_OK;
}
