// J1: int4 quantize-and-pack of 64-token temporal groups through the cross-loop
// residual chain (flashloop_torch/kv_quantization.py:395-414, 531-650).
//
// One workgroup (256 threads) encodes one group of one (batch, head) for all loops.
// K (per channel over 64 tokens) and V (per token over 64-channel halves) are
// independent chains, so each thread keeps the elements it owns in registers across
// loops and only the nibble transposition of K goes through LDS.
//
// Bit-exactness: every float op is a single IEEE op with explicit rounding
// (__fsub_rn/__fdiv_rn/__fmul_rn/__fadd_rn, no contraction), rintf is round-half-even,
// and bf16 narrowing is round-to-nearest-even -- the op sequence of the reference's
// eager torch-CPU codec.
#include "fl_common.h"

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
  float scale, minimum;
};

__device__ __forceinline__ Quant make_quant(float mn, float mx, bool any) {
  if (!any) {
    mn = 0.0f;
    mx = 0.0f;
  }
  const float span = __fsub_rn(mx, mn);
  const float scale = span > 0.0f ? __fdiv_rn(span, 15.0f) : 1.0f;
  return {scale, mn};
}

__device__ __forceinline__ uint32_t encode(float x, Quant q) {
  float c = rintf(__fdiv_rn(__fsub_rn(x, q.minimum), q.scale));
  c = fminf(fmaxf(c, 0.0f), 15.0f);
  return static_cast<uint32_t>(c);
}

__device__ __forceinline__ float decode(uint32_t code, Quant q) {
  return round_bf16(__fadd_rn(__fmul_rn(static_cast<float>(code), q.scale), q.minimum));
}

__device__ __forceinline__ bool row_active(const PackArgs& a, int r, int b, int src_row) {
  if (r < 2) return true;
  const uint8_t* m = a.mask[r - 2];
  return m == nullptr || m[static_cast<int64_t>(b) * a.mask_stride + src_row] != 0;
}

// destination row of logical token t in stream s (-1: not stored)
__device__ __forceinline__ int dst_row(const fl_cache_view& v, int s, int b, int t) {
  if (s < 2) return t;
  const int r = v.rank[s - 2][static_cast<int64_t>(b) * v.token_capacity + t];
  return r < v.row_capacity[s] ? r : -1;
}

__global__ __launch_bounds__(256) void pack_groups_kernel(PackArgs a) {
  const fl_cache_view& v = a.v;
  const int j = blockIdx.x;
  const int bh = blockIdx.y;
  const int b = bh / v.heads;
  const int g0 = a.dst_group0[b];
  if (g0 < 0) return;
  const int g = g0 + j;
  if ((g + 1) * kGroup > v.token_capacity) return;  // outside the destination

  const int tid = threadIdx.x;
  const int src_row0 = a.src_row_offset + j * kGroup;
  const int64_t src_base = (static_cast<int64_t>(bh) * a.src_bh_stride + src_row0) * kDim;

  __shared__ uint8_t codes_lds[kGroup][kRowBytes];

  // ------------------------------------------------------------------ K chain
  {
    const int pair = tid >> 2;     // channels 2*pair, 2*pair+1
    const int quarter = tid & 3;   // tokens quarter*16 .. +16
    float r0[16], r1[16];
    for (int r = 0; r < a.loops; ++r) {
      const int s = r;
      float x0[16], x1[16];
      bool act[16];
      float mn0 = INFINITY, mx0 = -INFINITY, mn1 = INFINITY, mx1 = -INFINITY;
      int nact = 0;
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const int i = quarter * 16 + k;
        const uint32_t w =
            *reinterpret_cast<const uint32_t*>(a.src_k[r] + src_base + static_cast<int64_t>(i) * kDim + 2 * pair);
        const float l0 = bf16lo_to_f32(w), l1 = bf16hi_to_f32(w);
        act[k] = row_active(a, r, b, src_row0 + i);
        if (r == 0) {
          x0[k] = l0;
          x1[k] = l1;
        } else {
          x0[k] = round_bf16(__fsub_rn(l0, r0[k]));
          x1[k] = round_bf16(__fsub_rn(l1, r1[k]));
        }
        if (act[k]) {
          mn0 = fminf(mn0, x0[k]);
          mx0 = fmaxf(mx0, x0[k]);
          mn1 = fminf(mn1, x1[k]);
          mx1 = fmaxf(mx1, x1[k]);
          ++nact;
        }
      }
      mn0 = quad_min(mn0);
      mx0 = quad_max(mx0);
      mn1 = quad_min(mn1);
      mx1 = quad_max(mx1);
      nact = quad_sum_i(nact);
      const Quant q0 = make_quant(mn0, mx0, nact > 0);
      const Quant q1 = make_quant(mn1, mx1, nact > 0);
      if (quarter == 0) {
        float4 meta = make_float4(q0.scale, q0.minimum, q1.scale, q1.minimum);
        const int64_t mi = ((static_cast<int64_t>(bh) * (v.token_capacity / kGroup) + g) * kDim + 2 * pair) * 2;
        *reinterpret_cast<float4*>(v.key_meta[s] + mi) = meta;
        const uint2 half_meta = make_uint2(
            static_cast<uint32_t>(f32_to_f16_sat(q0.scale)) | (static_cast<uint32_t>(f32_to_f16_sat(q0.minimum)) << 16),
            static_cast<uint32_t>(f32_to_f16_sat(q1.scale)) | (static_cast<uint32_t>(f32_to_f16_sat(q1.minimum)) << 16));
        *reinterpret_cast<uint2*>(v.key_meta_half[s] + mi) = half_meta;
      }
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const int i = quarter * 16 + k;
        uint32_t c0 = 0, c1 = 0;
        float d0 = 0.0f, d1 = 0.0f;
        if (act[k]) {
          c0 = encode(x0[k], q0);
          c1 = encode(x1[k], q1);
          d0 = decode(c0, q0);
          d1 = decode(c1, q1);
        }
        codes_lds[i][pair] = static_cast<uint8_t>(c0 | (c1 << 4));
        if (r == 0) {
          r0[k] = d0;
          r1[k] = d1;
        } else {
          // inactive rows add an exact zero delta (kv_quantization.py:465)
          r0[k] = round_bf16(__fadd_rn(r0[k], d0));
          r1[k] = round_bf16(__fadd_rn(r1[k], d1));
        }
        if (a.rk[r] != nullptr) {
          const uint32_t packed = static_cast<uint32_t>(f32_to_bf16_rne(r0[k])) |
                                  (static_cast<uint32_t>(f32_to_bf16_rne(r1[k])) << 16);
          *reinterpret_cast<uint32_t*>(a.rk[r] + src_base + static_cast<int64_t>(i) * kDim + 2 * pair) = packed;
        }
      }
      __syncthreads();
      {
        const int i = tid >> 2, chunk = tid & 3;
        const int t = g * kGroup + i;
        const int row = row_active(a, r, b, src_row0 + i) ? dst_row(v, s, b, t) : -1;
        if (row >= 0) {
          const uint4 val = *reinterpret_cast<const uint4*>(&codes_lds[i][chunk * 16]);
          *reinterpret_cast<uint4*>(v.key_codes[s] + (static_cast<int64_t>(bh) * v.row_capacity[s] + row) * kCodeStride +
                                    chunk * 16) = val;
        }
      }
      __syncthreads();
    }
  }

  // ------------------------------------------------------------------ V chain
  {
    const int i = tid >> 2;        // token row
    const int quarter = tid & 3;   // channels 32*quarter .. +32, half = quarter >> 1
    const int half = quarter >> 1;
    const int t = g * kGroup + i;
    const int64_t row_off = src_base + static_cast<int64_t>(i) * kDim + 32 * quarter;
    float rv[32];
    for (int r = 0; r < a.loops; ++r) {
      const int s = r;
      const bool act = row_active(a, r, b, src_row0 + i);
      float x[32];
      const uint4* src = reinterpret_cast<const uint4*>(a.src_v[r] + row_off);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint4 w = src[k];
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          x[8 * k + 2 * e] = bf16lo_to_f32(ws[e]);
          x[8 * k + 2 * e + 1] = bf16hi_to_f32(ws[e]);
        }
      }
      float mn = INFINITY, mx = -INFINITY;
#pragma unroll
      for (int c = 0; c < 32; ++c) {
        if (r > 0) x[c] = round_bf16(__fsub_rn(x[c], rv[c]));
        mn = fminf(mn, x[c]);
        mx = fmaxf(mx, x[c]);
      }
      mn = pair_min(mn);
      mx = pair_max(mx);
      const Quant q = make_quant(mn, mx, act);
      uint32_t words[4] = {0, 0, 0, 0};
#pragma unroll
      for (int c = 0; c < 32; ++c) {
        uint32_t code = 0;
        float d = 0.0f;
        if (act) {
          code = encode(x[c], q);
          d = decode(code, q);
        }
        words[c >> 3] |= code << (4 * (c & 7));
        rv[c] = (r == 0) ? d : round_bf16(__fadd_rn(rv[c], d));
      }
      const int row = act ? dst_row(v, s, b, t) : -1;
      if (row >= 0) {
        const int64_t rowi = static_cast<int64_t>(bh) * v.row_capacity[s] + row;
        *reinterpret_cast<uint4*>(v.value_codes[s] + rowi * kCodeStride + 16 * quarter) =
            make_uint4(words[0], words[1], words[2], words[3]);
        if ((quarter & 1) == 0) {
          *reinterpret_cast<float2*>(v.value_meta[s] + (rowi * 2 + half) * 2) = make_float2(q.scale, q.minimum);
          *reinterpret_cast<uint32_t*>(v.value_meta_half[s] + (rowi * 2 + half) * 2) =
              static_cast<uint32_t>(f32_to_f16_sat(q.scale)) | (static_cast<uint32_t>(f32_to_f16_sat(q.minimum)) << 16);
          const int64_t rec = ((static_cast<int64_t>(bh) * v.token_capacity + t) * 2 + half) * 4 + s;
          *reinterpret_cast<float2*>(v.value_meta_token + rec * 2) = make_float2(q.scale, q.minimum);
        }
      }
      if (a.rv[r] != nullptr) {
        uint4* dst = reinterpret_cast<uint4*>(a.rv[r] + row_off);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          uint32_t w[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            w[e] = static_cast<uint32_t>(f32_to_bf16_rne(rv[8 * k + 2 * e])) |
                   (static_cast<uint32_t>(f32_to_bf16_rne(rv[8 * k + 2 * e + 1])) << 16);
          }
          dst[k] = make_uint4(w[0], w[1], w[2], w[3]);
        }
      }
    }
  }
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
  dim3 grid(n_groups, v.batch * v.heads);
  hipLaunchKernelGGL(pack_groups_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream), a);
  FL_LAUNCH_CHECK("fl_pack_kv_groups");
  return FL_OK;
}
