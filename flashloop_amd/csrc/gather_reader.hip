// J2 (sparse): readers over a selected subset of keys of loop `loop`.
//
//  * fl_decode_attn_sparse_delta -- logits over the selected keys, subset softmax,
//    P.V, then the cached-mass correction mass*(target - source_output)
//    (flashloop/cache.py:1592-1617, flashloop_torch/attention_utils.py:216-248).
//  * fl_decode_selected_pv -- sum of given weights times the selected V rows
//    (flashloop/engine.py:346-371).
//
// A selected logical index is the current token (== packed + tail length), a tail row
// (>= packed length) or a packed prefix row; prefix rows are rebuilt from streams
// 0..loop, streams 2/3 through the rank maps.  Rows are token-major, so a selected
// token costs one 16-byte load per stream per channel quarter; its K metadata is the
// 1 KiB (scale, min) block of its 64-token group, which neighbouring selected tokens
// of the same group share through the caches.
//
// grid.x = chunk of kChunk selected slots, grid.y = (b,h).  Inside a workgroup,
// lane = 4*row + quarter as in the dense reader; each quad handles one selected slot
// per pass.  The workgroup max is known before P.V, so no online rescaling is needed.
#include "reader_common.h"

namespace fl {
namespace {
using namespace reader;

constexpr int kChunk = 256;  // selected slots per workgroup
constexpr int kQuads = kThreads / 4;

struct GatherArgs {
  fl_cache_view v;
  int loop;
  const uint16_t* q;
  const uint16_t* kc;
  const uint16_t* vc;
  const int32_t* idx;
  const uint8_t* valid;
  const float* weights;
  int cap;
  float scaling;
  float* ws;  // [B*H, nchunk, kPartial]
  int nchunk;
};

// physical row of logical prefix token t in stream s, or -1 (absent / out of capacity)
__device__ __forceinline__ int stream_row(const fl_cache_view& v, int s, int b, int t) {
  if (s < 2) return t;
  const int r = v.rank[s - 2][static_cast<int64_t>(b) * v.token_capacity + t];
  return r < v.row_capacity[s] ? r : -1;
}

// partial dot of q (LDS, pre-scaled) with the lane's 32 channels of a bf16 row
__device__ __forceinline__ float dot_bf16_row(const uint16_t* row, const float* qf, int quarter) {
  float d = 0.0f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint4 w = *reinterpret_cast<const uint4*>(row + 32 * quarter + 8 * k);
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      d = fmaf(qf[32 * quarter + 8 * k + 2 * e], bf16lo_to_f32(ws[e]), d);
      d = fmaf(qf[32 * quarter + 8 * k + 2 * e + 1], bf16hi_to_f32(ws[e]), d);
    }
  }
  return d;
}

__device__ __forceinline__ void axpy_bf16_row(const uint16_t* row, float p, int quarter, float* acc) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint4 w = *reinterpret_cast<const uint4*>(row + 32 * quarter + 8 * k);
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      acc[8 * k + 2 * e] = fmaf(p, bf16lo_to_f32(ws[e]), acc[8 * k + 2 * e]);
      acc[8 * k + 2 * e + 1] = fmaf(p, bf16hi_to_f32(ws[e]), acc[8 * k + 2 * e + 1]);
    }
  }
}

// MODE 0: subset softmax (sparse delta); MODE 1: given weights (selected PV)
template <int MODE>
__global__ __launch_bounds__(kThreads) void gather_reader_kernel(GatherArgs a) {
  const fl_cache_view& v = a.v;
  const int chunk = blockIdx.x;
  const int bh = blockIdx.y;
  const int b = bh / v.heads;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, quarter = lane & 3, row = lane >> 2;
  const int quad = wave * 16 + row;
  // lengths come from device memory: clamp them to the buffers so a bad value cannot fault
  const int Tp = min(v.packed_tokens[b], v.token_capacity) & ~(kGroup - 1);
  const int tl = min(v.tail_tokens[b], v.tail_capacity);
  const int cur = Tp + tl;
  const int gcap = v.token_capacity / kGroup;
  const int nst = a.loop + 1;

  __shared__ float qf[kDim];
  __shared__ float pw[kChunk];
  __shared__ float comb[kWaves][16][kDim];
  __shared__ float lsh[kWaves * 16];
  __shared__ float msh[kWaves];

  const int64_t sel0 = static_cast<int64_t>(bh) * a.cap + static_cast<int64_t>(chunk) * kChunk;
  const int nslots = min(kChunk, a.cap - chunk * kChunk);

  float M = 0.0f;
  if (MODE == 0) {
    if (tid < kDim) qf[tid] = bf16_to_f32(a.q[static_cast<int64_t>(bh) * kDim + tid]) * a.scaling;
    __syncthreads();
    for (int pass = 0; pass < kChunk / kQuads; ++pass) {
      const int slot = pass * kQuads + quad;
      bool ok = slot < nslots && a.valid[sel0 + slot] != 0;
      const int t = ok ? a.idx[sel0 + slot] : -1;
      ok = ok && t >= 0 && t <= cur;  // out-of-range indices are dropped, never read
      float d = 0.0f;
      if (ok) {
        if (t == cur) {
          d = dot_bf16_row(a.kc + static_cast<int64_t>(bh) * kDim, qf, quarter);
        } else if (t >= Tp) {
          d = dot_bf16_row(v.tail_key[a.loop] + (static_cast<int64_t>(bh) * v.tail_capacity + (t - Tp)) * kDim, qf,
                           quarter);
        } else {
          const int g = t / kGroup;
          for (int s = 0; s < nst; ++s) {
            const int r = stream_row(v, s, b, t);
            if (r < 0) continue;
            const uint4 w = *reinterpret_cast<const uint4*>(
                v.key_codes[s] + (static_cast<int64_t>(bh) * v.row_capacity[s] + r) * kRowBytes + 16 * quarter);
            const float4* meta = reinterpret_cast<const float4*>(
                v.key_meta[s] + ((static_cast<int64_t>(bh) * gcap + g) * kDim + 32 * quarter) * 2);
            const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                // byte e of word k: channels 8k+2e (low nibble), 8k+2e+1 (high nibble)
                const float4 sm = meta[4 * k + e];  // (scale, min) of both channels
                const int c = 32 * quarter + 8 * k + 2 * e;
                const float lo = static_cast<float>((ws[k] >> (8 * e)) & 0xFu);
                const float hi = static_cast<float>((ws[k] >> (8 * e + 4)) & 0xFu);
                d = fmaf(qf[c], fmaf(lo, sm.x, sm.y), d);
                d = fmaf(qf[c + 1], fmaf(hi, sm.z, sm.w), d);
              }
            }
          }
        }
      }
      d += shfl_xor(d, 1);
      d += shfl_xor(d, 2);
      if (quarter == 0) pw[slot] = ok ? d : -INFINITY;
    }
    __syncthreads();
    const float mt = wave_max(pw[tid]);
    if (lane == 0) msh[wave] = mt;
    __syncthreads();
    M = fmaxf(fmaxf(msh[0], msh[1]), fmaxf(msh[2], msh[3]));
    const float l = pw[tid];
    pw[tid] = (l == -INFINITY) ? 0.0f : fast_exp2((l - M) * kLog2e);
    __syncthreads();
  } else {
    bool ok = tid < nslots && a.valid[sel0 + tid] != 0;
    if (ok) {
      const int t = a.idx[sel0 + tid];
      ok = t >= 0 && t <= cur;
    }
    pw[tid] = ok ? a.weights[sel0 + tid] : 0.0f;
    __syncthreads();
  }

  float acc[32];
#pragma unroll
  for (int c = 0; c < 32; ++c) acc[c] = 0.0f;
  float mu = 0.0f, lsum = 0.0f;
  for (int pass = 0; pass < kChunk / kQuads; ++pass) {
    const int slot = pass * kQuads + quad;
    const float p = pw[slot];
    if (p == 0.0f) continue;
    lsum += p;
    const int t = a.idx[sel0 + slot];
    if (t == cur) {
      axpy_bf16_row(a.vc + static_cast<int64_t>(bh) * kDim, p, quarter, acc);
    } else if (t >= Tp) {
      axpy_bf16_row(v.tail_value[a.loop] + (static_cast<int64_t>(bh) * v.tail_capacity + (t - Tp)) * kDim, p, quarter,
                    acc);
    } else {
      for (int s = 0; s < nst; ++s) {
        const int r = stream_row(v, s, b, t);
        if (r < 0) continue;
        const int64_t rowi = static_cast<int64_t>(bh) * v.row_capacity[s] + r;
        const uint4 w = *reinterpret_cast<const uint4*>(v.value_codes[s] + rowi * kRowBytes + 16 * quarter);
        const float2 sm = *reinterpret_cast<const float2*>(v.value_meta[s] + (rowi * 2 + (quarter >> 1)) * 2);
        const float we = p * sm.x;
        mu = fmaf(p, sm.y, mu);
        axpy8(w.x, we, we * 0.0625f, acc + 0);
        axpy8(w.y, we, we * 0.0625f, acc + 8);
        axpy8(w.z, we, we * 0.0625f, acc + 16);
        axpy8(w.w, we, we * 0.0625f, acc + 24);
      }
    }
  }
  // combine the quads (common max M already applied through p)
#pragma unroll
  for (int c = 0; c < 32; ++c) comb[wave][row][32 * quarter + c] = acc[c] + mu;
  if (quarter == 0) lsh[wave * 16 + row] = lsum;
  __syncthreads();
  float* part = a.ws + (static_cast<int64_t>(bh) * a.nchunk + chunk) * kPartial;
  if (tid < kDim) {
    float s = 0.0f;
    for (int w = 0; w < kWaves; ++w)
      for (int r = 0; r < 16; ++r) s += comb[w][r][tid];
    part[2 + tid] = s;
  } else if (tid == kDim) {
    float s = 0.0f;
    for (int i = 0; i < kWaves * 16; ++i) s += lsh[i];
    part[0] = (MODE == 0 && s == 0.0f) ? -INFINITY : M;
    part[1] = s;
  }
}

int32_t check_gather_args(const fl_cache_view* view, int32_t loop, const int32_t* indices, const uint8_t* valid,
                          int32_t capacity, void* workspace, size_t workspace_bytes, size_t need, const char* who) {
  FL_REQUIRE(view != nullptr, std::string(who) + ": view is null");
  const fl_cache_view& v = *view;
  FL_REQUIRE(loop >= 0 && loop <= 3, std::string(who) + ": loop must be in 0..3");
  FL_REQUIRE(indices && valid && workspace, std::string(who) + ": null indices/valid/workspace");
  FL_REQUIRE(capacity > 0, std::string(who) + ": capacity must be positive");
  FL_REQUIRE(v.batch > 0 && v.heads > 0 && v.token_capacity % kGroup == 0, std::string(who) + ": bad view geometry");
  FL_REQUIRE(v.packed_tokens && v.tail_tokens, std::string(who) + ": null length arrays");
  FL_REQUIRE(v.tail_key[loop] && v.tail_value[loop], std::string(who) + ": null tail for this loop");
  for (int s = 0; s <= loop && v.max_packed_tokens > 0; ++s) {
    FL_REQUIRE(v.key_codes[s] && v.key_meta[s] && v.value_codes[s] && v.value_meta[s],
               std::string(who) + ": null stream pointer");
    if (s >= 2) FL_REQUIRE(v.rank[s - 2] != nullptr, std::string(who) + ": null rank map");
  }
  FL_REQUIRE(workspace_bytes >= need, std::string(who) + ": workspace too small");
  return FL_OK;
}

}  // namespace
}  // namespace fl

extern "C" size_t fl_decode_selected_workspace(const fl_cache_view* view, int32_t capacity) {
  using namespace fl;
  if (!view || capacity <= 0) return 0;
  const int nchunk = (capacity + kChunk - 1) / kChunk;
  return static_cast<size_t>(view->batch) * view->heads * nchunk * kPartial * sizeof(float);
}

extern "C" int32_t fl_decode_selected_pv(const fl_cache_view* view, int32_t loop, const int32_t* indices,
                                         const uint8_t* valid, const float* weights, int32_t capacity,
                                         const uint16_t* v_cur, float* out, void* workspace, size_t workspace_bytes,
                                         void* stream) {
  using namespace fl;
  clear_error();
  const int32_t rc = check_gather_args(view, loop, indices, valid, capacity, workspace, workspace_bytes,
                                       fl_decode_selected_workspace(view, capacity), "fl_decode_selected_pv");
  if (rc != FL_OK) return rc;
  FL_REQUIRE(weights && v_cur && out, "fl_decode_selected_pv: null weights/v_cur/out");
  GatherArgs a{};
  a.v = *view;
  a.loop = loop;
  a.vc = v_cur;
  a.idx = indices;
  a.valid = valid;
  a.weights = weights;
  a.cap = capacity;
  a.ws = static_cast<float*>(workspace);
  a.nchunk = (capacity + kChunk - 1) / kChunk;
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(gather_reader_kernel<1>, dim3(a.nchunk, view->batch * view->heads), dim3(kThreads), 0, st, a);
  FL_LAUNCH_CHECK("fl_decode_selected_pv(reader)");
  hipLaunchKernelGGL(merge_partials_kernel, dim3(view->batch * view->heads), dim3(kDim), 0, st,
                     static_cast<const float*>(a.ws), a.nchunk, out, kMergeSum, static_cast<const float*>(nullptr),
                     static_cast<const float*>(nullptr));
  FL_LAUNCH_CHECK("fl_decode_selected_pv(merge)");
  return FL_OK;
}

extern "C" int32_t fl_decode_attn_sparse_delta(const fl_cache_view* view, int32_t loop, const uint16_t* q,
                                               const uint16_t* k_cur, const uint16_t* v_cur, const int32_t* indices,
                                               const uint8_t* valid, int32_t capacity, const float* source_output,
                                               const float* mass, float scaling, float* out, void* workspace,
                                               size_t workspace_bytes, void* stream) {
  using namespace fl;
  clear_error();
  const int32_t rc = check_gather_args(view, loop, indices, valid, capacity, workspace, workspace_bytes,
                                       fl_decode_selected_workspace(view, capacity), "fl_decode_attn_sparse_delta");
  if (rc != FL_OK) return rc;
  FL_REQUIRE(q && k_cur && v_cur && source_output && mass && out,
             "fl_decode_attn_sparse_delta: null vector/output pointer");
  GatherArgs a{};
  a.v = *view;
  a.loop = loop;
  a.q = q;
  a.kc = k_cur;
  a.vc = v_cur;
  a.idx = indices;
  a.valid = valid;
  a.cap = capacity;
  a.scaling = scaling;
  a.ws = static_cast<float*>(workspace);
  a.nchunk = (capacity + kChunk - 1) / kChunk;
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(gather_reader_kernel<0>, dim3(a.nchunk, view->batch * view->heads), dim3(kThreads), 0, st, a);
  FL_LAUNCH_CHECK("fl_decode_attn_sparse_delta(reader)");
  hipLaunchKernelGGL(merge_partials_kernel, dim3(view->batch * view->heads), dim3(kDim), 0, st,
                     static_cast<const float*>(a.ws), a.nchunk, out, kMergeMassDelta, mass, source_output);
  FL_LAUNCH_CHECK("fl_decode_attn_sparse_delta(merge)");
  return FL_OK;
}
