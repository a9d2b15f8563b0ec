// J2: fused dense decode reader over the packed int4 residual cache.
//
// logit_t = scaling * q . K_loop[t],  K_loop[t] = sum_{s<=loop} deq(stream s)[t]
// out     = softmax(logits) . V_loop  over [packed prefix ; BF16 tail ; current token]
//
// Layout of the work (one launch + a merge launch):
//   grid.x = split index (nsplit prefix splits + 1 tail/current split), grid.y = (b,h).
//   A prefix split owns `gps` consecutive 64-token groups.  Each wave takes one group
//   per iteration; inside a wave, lane = 4*row + quarter: 16 token rows x 4 channel
//   quarters (32 channels = one 16-byte load per stream per token).
//
// Per-channel K metadata is factored out of the dot product: for group g and stream s,
//   q . deq_s(K)[t] = sum_c (q_c*scale_{g,c}) * code_{t,c} + sum_c q_c*min_{g,c},
// so a token costs one nibble convert and one FMA per channel per stream; the
// q*scale products and the min term are built once per group per wave in LDS.
// Likewise V (per-token metadata) is accumulated as
//   sum_t p_t*(scale_t*code_t,c + min_t) = sum_t (p_t*scale_t)*code_t,c + sum_t p_t*min_t.
// Each 4-lane quad keeps its own online-softmax state; the 64 quad states of a
// workgroup are merged through LDS at the end of the split, and the splits of a row by
// a second kernel.  No MFMA: one query per head makes this a GEMV, bound by HBM.
#include "reader_common.h"

namespace fl {
namespace {
using namespace reader;

struct DenseArgs {
  fl_cache_view v;
  int loop;
  const uint16_t* q;
  const uint16_t* kc;
  const uint16_t* vc;
  float scaling;
  float* logits;
  int64_t logits_stride;
  float* ws;  // [B*H, nsplit+1, kPartial]
  float* out;
  const uint16_t* tail_k;  // tail_key[loop] / tail_value[loop], resolved on the host
  const uint16_t* tail_v;
  int nsplit;
  int gps;    // groups per prefix split
};

// Registers of one half-group (32 tokens, 2 per lane): K/V codes and V metadata of
// every stream, plus (first half only) the group's K metadata for this lane's 2 channels.
template <int NS>
struct HalfSet {
  float4 kmeta[NS];
  uint4 kw[2][NS];
  uint4 vw[2][NS];
  float2 vm[2][NS];
  bool has[2][NS];
};

template <int NS>
__device__ __forceinline__ void load_half(HalfSet<NS>& hs, const fl_cache_view& v, int bh, int b, int gi, int h,
                                          int row, int quarter, int gcap) {
  const int lane = threadIdx.x & 63;
  if (h == 0) {
#pragma unroll
    for (int s = 0; s < NS; ++s)
      hs.kmeta[s] = *reinterpret_cast<const float4*>(
          v.key_meta[s] + ((static_cast<int64_t>(bh) * gcap + gi) * kDim + 2 * lane) * 2);
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int t = gi * kGroup + row + 16 * (2 * h + i);
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      int r = t;
      if (s >= 2) r = v.rank[s - 2][static_cast<int64_t>(b) * v.token_capacity + t];
      hs.has[i][s] = r >= 0 && r < v.row_capacity[s];
      if (!hs.has[i][s]) r = 0;
      const int64_t rowi = static_cast<int64_t>(bh) * v.row_capacity[s] + r;
      hs.kw[i][s] = *reinterpret_cast<const uint4*>(v.key_codes[s] + rowi * kRowBytes + 16 * quarter);
      hs.vw[i][s] = *reinterpret_cast<const uint4*>(v.value_codes[s] + rowi * kRowBytes + 16 * quarter);
      hs.vm[i][s] = *reinterpret_cast<const float2*>(v.value_meta[s] + (rowi * 2 + (quarter >> 1)) * 2);
    }
  }
}

// Logits, online softmax and P.V for one half-group.  At h == 0 the group's q*scale
// products (LDS, wave-private) and q.min constants are rebuilt from hs.kmeta.
template <int NS>
__device__ __forceinline__ void dense_half(HalfSet<NS>& hs, QuadState& st, const DenseArgs& a, const float* qf,
                                           float (*qsh)[kDim], int b, int gi, int h, int row, int quarter,
                                           float* lrow) {
  const int lane = threadIdx.x & 63;
  __shared__ float cs_sh[kWaves][4];
  float* cs = cs_sh[threadIdx.x >> 6];
  if (h == 0) {
    const float q0 = qf[2 * lane], q1 = qf[2 * lane + 1];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      qsh[s][2 * lane] = q0 * hs.kmeta[s].x;
      qsh[s][2 * lane + 1] = q1 * hs.kmeta[s].z * 0.0625f;  // odd channel: high nibble reads 16*code
      const float c = wave_sum(fmaf(q0, hs.kmeta[s].y, q1 * hs.kmeta[s].w));
      if (lane == 0) cs[s] = c;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  float lg[2] = {0.0f, 0.0f};
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    float qe[16], qo[16];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float4 x = *reinterpret_cast<const float4*>(&qsh[s][32 * quarter + 8 * k]);
      const float4 y = *reinterpret_cast<const float4*>(&qsh[s][32 * quarter + 8 * k + 4]);
      qe[4 * k + 0] = x.x; qo[4 * k + 0] = x.y;
      qe[4 * k + 1] = x.z; qo[4 * k + 1] = x.w;
      qe[4 * k + 2] = y.x; qo[4 * k + 2] = y.y;
      qe[4 * k + 3] = y.z; qo[4 * k + 3] = y.w;
    }
    const float c = cs[s];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      float d = 0.0f;
      d = dot8(hs.kw[i][s].x, qe + 0, qo + 0, d);
      d = dot8(hs.kw[i][s].y, qe + 4, qo + 4, d);
      d = dot8(hs.kw[i][s].z, qe + 8, qo + 8, d);
      d = dot8(hs.kw[i][s].w, qe + 12, qo + 12, d);
      d = quad_sum(d) + c;
      if (s < 2 || hs.has[i][s]) lg[i] += d;
    }
  }
  if (lrow && quarter == 0) {
    lrow[gi * kGroup + row + 16 * (2 * h)] = lg[0];
    lrow[gi * kGroup + row + 16 * (2 * h + 1)] = lg[1];
  }
  float p[2];
  online_update(st, lg, p, 2);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      if (s >= 2 && !hs.has[i][s]) continue;
      const float we = p[i] * hs.vm[i][s].x;
      const float wo = we * 0.0625f;
      st.mu = fmaf(p[i], hs.vm[i][s].y, st.mu);
      axpy8(hs.vw[i][s].x, we, wo, st.acc + 0);
      axpy8(hs.vw[i][s].y, we, wo, st.acc + 8);
      axpy8(hs.vw[i][s].z, we, wo, st.acc + 16);
      axpy8(hs.vw[i][s].w, we, wo, st.acc + 24);
    }
  }
}

template <int NS>
__global__ __launch_bounds__(kThreads) void dense_reader_kernel(DenseArgs a) {
  const fl_cache_view& v = a.v;
  const int split = blockIdx.x;
  const int bh = blockIdx.y;
  const int b = bh / v.heads;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, quarter = lane & 3, row = lane >> 2;
  // lengths come from device memory: clamp them to the buffers so a bad value cannot fault
  const int Tp = min(v.packed_tokens[b], v.token_capacity) & ~(kGroup - 1);
  const int tl = min(v.tail_tokens[b], v.tail_capacity);

  __shared__ float qf[kDim];
  __shared__ float qsh[kWaves][NS][kDim];
  __shared__ float comb[kWaves][16][kDim];
  __shared__ float lsh[kWaves * 16];
  __shared__ float msh[kWaves];

  if (tid < kDim) qf[tid] = bf16_to_f32(a.q[static_cast<int64_t>(bh) * kDim + tid]) * a.scaling;
  __syncthreads();

  QuadState st;
  st.m = -INFINITY;
  st.l = 0.0f;
  st.mu = 0.0f;
#pragma unroll
  for (int c = 0; c < 32; ++c) st.acc[c] = 0.0f;

  float* part = a.ws + (static_cast<int64_t>(bh) * (a.nsplit + 1) + split) * kPartial;
  float* lrow = a.logits ? a.logits + static_cast<int64_t>(bh) * a.logits_stride : nullptr;

  if (split < a.nsplit) {
    const int G = Tp / kGroup;
    const int g_begin = split * a.gps;
    const int g_end = min(g_begin + a.gps, G);
    const int gcap = v.token_capacity / kGroup;
    // This wave's work: groups g_begin+wave, +kWaves, ... each as two half-groups of 32
    // tokens (2 per lane).  Unit u = 2*k + h covers half h of the wave's k-th group.
    const int my_groups = (g_end - g_begin - wave + kWaves - 1) / kWaves;
    const int units = g_end - g_begin > wave ? 2 * my_groups : 0;
    HalfSet<NS> set0, set1;
    if (units > 0) load_half<NS>(set0, v, bh, b, g_begin + wave, 0, row, quarter, gcap);
    for (int u = 0; u < units; u += 2) {
      // ping-pong: the next unit's loads are in flight while this one computes
      load_half<NS>(set1, v, bh, b, g_begin + wave + (u >> 1) * kWaves, 1, row, quarter, gcap);
      dense_half<NS>(set0, st, a, qf, qsh[wave], b, g_begin + wave + (u >> 1) * kWaves, 0, row, quarter, lrow);
      if (u + 2 < units) load_half<NS>(set0, v, bh, b, g_begin + wave + ((u >> 1) + 1) * kWaves, 0, row, quarter, gcap);
      dense_half<NS>(set1, st, a, qf, qsh[wave], b, g_begin + wave + (u >> 1) * kWaves, 1, row, quarter, lrow);
    }
  } else {
    // ---- BF16 tail of this loop, then the current token (virtual row tl)
    const uint16_t* tk = a.tail_k + static_cast<int64_t>(bh) * v.tail_capacity * kDim;
    const uint16_t* tv = a.tail_v + static_cast<int64_t>(bh) * v.tail_capacity * kDim;
    const uint16_t* ck = a.kc + static_cast<int64_t>(bh) * kDim;
    const uint16_t* cv = a.vc + static_cast<int64_t>(bh) * kDim;
    float qr[32];
#pragma unroll
    for (int c = 0; c < 32; ++c) qr[c] = qf[32 * quarter + c];
    const int n = tl + 1;
    for (int base = wave * 16; base < n; base += kWaves * 16) {
      const int vt = base + row;
      const bool valid = vt < n;
      const uint16_t* kr = (vt < tl) ? tk + static_cast<int64_t>(vt) * kDim : ck;
      const uint16_t* vr = (vt < tl) ? tv + static_cast<int64_t>(vt) * kDim : cv;
      float d = 0.0f;
      uint4 vwords[4];
      if (valid) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint4 w = *reinterpret_cast<const uint4*>(kr + 32 * quarter + 8 * k);
          d = fmaf(qr[8 * k + 0], bf16lo_to_f32(w.x), d);
          d = fmaf(qr[8 * k + 1], bf16hi_to_f32(w.x), d);
          d = fmaf(qr[8 * k + 2], bf16lo_to_f32(w.y), d);
          d = fmaf(qr[8 * k + 3], bf16hi_to_f32(w.y), d);
          d = fmaf(qr[8 * k + 4], bf16lo_to_f32(w.z), d);
          d = fmaf(qr[8 * k + 5], bf16hi_to_f32(w.z), d);
          d = fmaf(qr[8 * k + 6], bf16lo_to_f32(w.w), d);
          d = fmaf(qr[8 * k + 7], bf16hi_to_f32(w.w), d);
          vwords[k] = *reinterpret_cast<const uint4*>(vr + 32 * quarter + 8 * k);
        }
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) vwords[k] = make_uint4(0, 0, 0, 0);
      }
      d = quad_sum(d);
      float lg = valid ? d : -INFINITY;
      if (lrow && quarter == 0 && valid) lrow[Tp + vt] = lg;
      float p;
      online_update(st, &lg, &p, 1);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t ws[4] = {vwords[k].x, vwords[k].y, vwords[k].z, vwords[k].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          st.acc[8 * k + 2 * e] = fmaf(p, bf16lo_to_f32(ws[e]), st.acc[8 * k + 2 * e]);
          st.acc[8 * k + 2 * e + 1] = fmaf(p, bf16hi_to_f32(ws[e]), st.acc[8 * k + 2 * e + 1]);
        }
      }
    }
  }
  write_partial(st, part, comb, lsh, msh);
}

int choose_gps(const fl_cache_view& v) {
  const int64_t rows = static_cast<int64_t>(v.batch) * v.heads;
  const int64_t groups = v.max_packed_tokens / kGroup;
  const int64_t target_blocks = 2048;
  int64_t gps = (groups * rows + target_blocks - 1) / target_blocks;
  gps = ((gps + kWaves - 1) / kWaves) * kWaves;  // whole iterations for every wave
  if (gps < kWaves) gps = kWaves;
  if (gps > 64) gps = 64;
  return static_cast<int>(gps);
}

int nsplit_of(const fl_cache_view& v, int gps) {
  const int groups = v.max_packed_tokens / kGroup;
  return (groups + gps - 1) / gps;
}

}  // namespace
}  // namespace fl

extern "C" size_t fl_decode_attn_dense_workspace(const fl_cache_view* view) {
  using namespace fl;
  if (!view) return 0;
  const int gps = choose_gps(*view);
  const int ns = nsplit_of(*view, gps);
  const int rows = view->batch * view->heads;
  return static_cast<size_t>(rows) * (ns + 1) * kPartial * sizeof(float);
}

extern "C" int32_t fl_decode_attn_dense(const fl_cache_view* view, int32_t loop, const uint16_t* q,
                                        const uint16_t* k_cur, const uint16_t* v_cur, float scaling, float* out,
                                        float* logits, int64_t logits_stride, void* workspace,
                                        size_t workspace_bytes, void* stream) {
  using namespace fl;
  clear_error();
  FL_REQUIRE(view != nullptr, "fl_decode_attn_dense: view is null");
  const fl_cache_view& v = *view;
  FL_REQUIRE(loop >= 0 && loop <= 3, "fl_decode_attn_dense: loop must be in 0..3");
  FL_REQUIRE(q && k_cur && v_cur && out && workspace, "fl_decode_attn_dense: null vector/output/workspace");
  FL_REQUIRE(v.batch > 0 && v.heads > 0 && v.token_capacity % kGroup == 0, "fl_decode_attn_dense: bad view geometry");
  FL_REQUIRE(v.max_packed_tokens >= 0 && v.max_packed_tokens <= v.token_capacity && v.max_packed_tokens % kGroup == 0,
             "fl_decode_attn_dense: max_packed_tokens must be a multiple of 64 within token_capacity");
  FL_REQUIRE(v.max_tail_tokens >= 0 && v.max_tail_tokens <= v.tail_capacity,
             "fl_decode_attn_dense: max_tail_tokens exceeds tail_capacity");
  FL_REQUIRE(v.packed_tokens && v.tail_tokens, "fl_decode_attn_dense: null length arrays");
  FL_REQUIRE(v.tail_key[loop] && v.tail_value[loop], "fl_decode_attn_dense: null tail for this loop");
  for (int s = 0; s <= loop && v.max_packed_tokens > 0; ++s) {
    FL_REQUIRE(v.key_codes[s] && v.key_meta[s] && v.value_codes[s] && v.value_meta[s],
               "fl_decode_attn_dense: null stream pointer");
    if (s >= 2) FL_REQUIRE(v.rank[s - 2] != nullptr, "fl_decode_attn_dense: null rank map");
  }
  FL_REQUIRE(logits == nullptr || logits_stride >= static_cast<int64_t>(v.max_packed_tokens) + v.max_tail_tokens + 1,
             "fl_decode_attn_dense: logits_stride smaller than the key count");
  FL_REQUIRE(workspace_bytes >= fl_decode_attn_dense_workspace(view), "fl_decode_attn_dense: workspace too small");
  FL_REQUIRE(nsplit_of(v, choose_gps(v)) + 1 <= kMergeMaxParts, "fl_decode_attn_dense: context too long for one merge");
  FL_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 16 == 0, "fl_decode_attn_dense: workspace must be 16-byte aligned");
  DenseArgs a{};
  a.v = v;
  a.loop = loop;
  a.q = q;
  a.kc = k_cur;
  a.vc = v_cur;
  a.scaling = scaling;
  a.logits = logits;
  a.logits_stride = logits_stride;
  a.ws = static_cast<float*>(workspace);
  a.gps = choose_gps(v);
  a.nsplit = nsplit_of(v, a.gps);
  a.out = out;
  a.tail_k = v.tail_key[loop];
  a.tail_v = v.tail_value[loop];
  const dim3 grid(a.nsplit + 1, v.batch * v.heads);
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (loop) {
    case 0: hipLaunchKernelGGL(dense_reader_kernel<1>, grid, dim3(kThreads), 0, st, a); break;
    case 1: hipLaunchKernelGGL(dense_reader_kernel<2>, grid, dim3(kThreads), 0, st, a); break;
    case 2: hipLaunchKernelGGL(dense_reader_kernel<3>, grid, dim3(kThreads), 0, st, a); break;
    default: hipLaunchKernelGGL(dense_reader_kernel<4>, grid, dim3(kThreads), 0, st, a); break;
  }
  FL_LAUNCH_CHECK("fl_decode_attn_dense(reader)");
  hipLaunchKernelGGL(merge_partials_kernel, dim3(v.batch * v.heads), dim3(kDim), 0, st,
                     static_cast<const float*>(a.ws), a.nsplit + 1, out, static_cast<int>(kMergeSoftmax),
                     static_cast<const float*>(nullptr), static_cast<const float*>(nullptr),
                     static_cast<const float*>(nullptr), static_cast<float*>(nullptr));
  FL_LAUNCH_CHECK("fl_decode_attn_dense(merge)");
  return FL_OK;
}
