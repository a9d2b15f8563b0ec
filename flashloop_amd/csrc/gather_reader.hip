// J2 (sparse): readers over a selected subset of keys of loop `loop`.
//
//  * fl_decode_attn_sparse_delta -- logits over the selected keys, subset softmax,
//    P.V, then the cached-mass correction mass*(target - source_output)
//    (flashloop/cache.py:1592-1617, flashloop_torch/attention_utils.py:216-248).
//    Optionally it also forms the loop-2 selected aggregate source_output itself
//    (flashloop/engine.py:346-371) from the V rows it reads anyway.
//  * fl_decode_selected_pv -- sum of given weights times the selected V rows
//    (flashloop/engine.py:346-371).
//
// A selected logical index is the current token (== packed + tail length), a tail row
// (>= packed length) or a packed prefix row; prefix rows are rebuilt from streams
// 0..loop, streams 2/3 through the rank maps.
//
// One workgroup owns kSlots consecutive selection slots, one 4-lane quad per slot
// (lane = 4*quad_row + quarter, 32 channels per lane).  The K metadata of a 64-token
// group is 1 KiB per stream and is shared by every selected token of that group (about
// six at 10% selection), so it is read once per workgroup: slots are grouped into runs
// of equal group (wave ballots), and each run's q*scale products and q.min constant are
// staged in LDS before the quads take their dot products, as in the dense reader.
// The workgroup's partial (max, sum, acc[128]) goes to the workspace; a small merge
// kernel combines a row's partials.
#include "reader_common.h"

namespace fl {
namespace {
using namespace reader;

constexpr int kSlots = 64;  // selection slots per workgroup (one quad each)
constexpr int kWin = 8;     // group runs whose K metadata is staged at once (a multiple of 4)

enum GatherMode { kSparseDelta = 0, kSelectedPV = 1, kSparseDeltaFused = 2 };

struct GatherArgs {
  fl_cache_view v;
  int loop;
  const uint16_t* q;
  const uint16_t* kc;
  const uint16_t* vc;
  const int32_t* idx;
  const uint8_t* valid;
  const float* weights;   // selected weights (kSelectedPV, kSparseDeltaFused)
  const uint16_t* vc1;    // loop-2 current value (kSparseDeltaFused)
  const uint16_t* tail_k;  // tail_key[loop] / tail_value[loop] / tail_value[1], resolved on the host
  const uint16_t* tail_v;
  const uint16_t* tail_v1;
  int cap;
  float scaling;
  float* ws;              // [B*H, nchunk, kPartial] (+ second set for the fused source aggregate)
  int nchunk;
  float* out;
  const float* mass;
  const float* src;       // source_output (kSparseDelta)
  float* src_out;         // source_output written (kSparseDeltaFused)
};

__device__ __forceinline__ void axpy_bf16_words(uint4 w, float p, float* acc) {
  const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    acc[2 * e] = fmaf(p, bf16lo_to_f32(ws[e]), acc[2 * e]);
    acc[2 * e + 1] = fmaf(p, bf16hi_to_f32(ws[e]), acc[2 * e + 1]);
  }
}

__device__ __forceinline__ float dot_bf16_words(uint4 w, const float* q) {
  float d = 0.0f;
  const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    d = fmaf(q[2 * e], bf16lo_to_f32(ws[e]), d);
    d = fmaf(q[2 * e + 1], bf16hi_to_f32(ws[e]), d);
  }
  return d;
}

#ifndef FL_GATHER_MIN_BLOCKS
#define FL_GATHER_MIN_BLOCKS 1
#endif
template <int NS, int MODE>
__global__ __launch_bounds__(kThreads, FL_GATHER_MIN_BLOCKS) void gather_reader_kernel(GatherArgs a) {
  const fl_cache_view& v = a.v;
  const int chunk = blockIdx.x;
  const int bh = blockIdx.y;
  const int b = bh / v.heads;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, quarter = lane & 3;
  const int quad = tid >> 2;  // selection slot of this quad
  // lengths come from device memory: clamp them to the buffers so a bad value cannot fault
  const int Tp = min(v.packed_tokens[b], v.token_capacity) & ~(kGroup - 1);
  const int tl = min(v.tail_tokens[b], v.tail_capacity);
  const int cur = Tp + tl;
  const int gcap = v.token_capacity / kGroup;
  constexpr bool kSoftmax = MODE != kSelectedPV;
  constexpr bool kSource = MODE == kSparseDeltaFused;

  __shared__ float qf[kDim];
  __shared__ int tok[kSlots];
  __shared__ int run_of[kSlots];
  __shared__ int run_group[kSlots];
  __shared__ int rows_sh[kSlots][NS];
  __shared__ float pw[kSlots];
  __shared__ float sw[kSlots];
  // q*scale staging (logit phase) and the quad merge (end) never overlap: one LDS block
  constexpr int kStage = kWin * NS * kDim + kWin * NS;
  constexpr int kComb = kWaves * 16 * kDim;
  __shared__ float lds_union[kStage > kComb ? kStage : kComb];
  float(*qsh)[NS][kDim] = reinterpret_cast<float(*)[NS][kDim]>(lds_union);
  float(*csh)[NS] = reinterpret_cast<float(*)[NS]>(lds_union + kWin * NS * kDim);
  float(*comb)[16][kDim] = reinterpret_cast<float(*)[16][kDim]>(lds_union);
  __shared__ float lsh[kWaves * 16];
  __shared__ float msh[kWaves];
  __shared__ int n_runs;

  const int64_t sel0 = static_cast<int64_t>(bh) * a.cap + static_cast<int64_t>(chunk) * kSlots;
  const int nslots = min(kSlots, a.cap - chunk * kSlots);

  // ---- slot table: logical token, physical stream rows, runs of equal group (wave 0)
  if (wave == 0) {
    int t = -1;
    if (lane < nslots) {  // index and flag loads issued together
      const int ti = a.idx[sel0 + lane];
      const bool ok = a.valid[sel0 + lane] != 0;
      t = (ok && ti >= 0 && ti <= cur) ? ti : -1;  // out-of-range indices are dropped, never read
    }
    tok[lane] = t;
    const bool pre = t >= 0 && t < Tp;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      int r = -1;
      if (pre) {
        if (s < 2) {
          r = t;
        } else {
          r = v.rank[s - 2][static_cast<int64_t>(b) * v.token_capacity + t];
          if (r >= v.row_capacity[s]) r = -1;
        }
      }
      rows_sh[lane][s] = r;
    }
    const int g = pre ? t / kGroup : -1;
    const int gprev = __shfl_up(g, 1, kWave);
    const bool start = pre && (lane == 0 || gprev != g);
    const uint64_t starts = __ballot(start);
    const uint64_t le_mask = (lane == 63) ? ~0ull : ((2ull << lane) - 1);
    const int run = pre ? __popcll(starts & le_mask) - 1 : -1;
    run_of[lane] = run;
    if (start) run_group[run] = g;
    if (lane == 0) n_runs = __popcll(starts);
    if (kSource) sw[lane] = (t >= 0) ? a.weights[sel0 + lane] : 0.0f;
    if (MODE == kSelectedPV) pw[lane] = (t >= 0) ? a.weights[sel0 + lane] : 0.0f;
  }
  if (kSoftmax && tid < kDim) qf[tid] = bf16_to_f32(a.q[static_cast<int64_t>(bh) * kDim + tid]) * a.scaling;
  lds_barrier();

  const int t = tok[quad];
  const int run = run_of[quad];
  int rows[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) rows[s] = rows_sh[quad][s];

  // Loads are issued in the order they are consumed -- K codes, the first window's K
  // metadata, then the V rows -- because the memory counter retires in issue order:
  // waiting for K must not also drain the V loads.
  const bool is_pre = run >= 0;
  const bool is_bf16 = t >= Tp;  // tail row or current token
  constexpr int kRunsPerWave = kWin / kWaves;
  const int nr = n_runs;
  uint4 kw[NS];
  float4 meta[kRunsPerWave][NS];
  auto load_meta = [&](int w0) {
    const int nw = min(kWin, nr - w0);
#pragma unroll
    for (int j = 0; j < kRunsPerWave; ++j) {
      const int wr = wave + kWaves * j;
      const int g = wr < nw ? run_group[w0 + wr] : 0;
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        meta[j][s] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (wr < nw)
          meta[j][s] = *reinterpret_cast<const float4*>(
              v.key_meta[s] + ((static_cast<int64_t>(bh) * gcap + g) * kDim + 2 * lane) * 2);
      }
    }
  };
  if (kSoftmax) {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      kw[s] = make_uint4(0, 0, 0, 0);
      if (is_pre && rows[s] >= 0)
        kw[s] = *reinterpret_cast<const uint4*>(
            v.key_codes[s] + (static_cast<int64_t>(bh) * v.row_capacity[s] + rows[s]) * kCodeStride + 16 * quarter);
    }
    if (nr > 0) load_meta(0);
  }
  uint4 vw[NS];
  float2 vm[NS];
  uint4 vbf[4];  // bf16 tail / current row (32 channels)
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    vw[s] = make_uint4(0, 0, 0, 0);
    vm[s] = make_float2(0.0f, 0.0f);
    if (is_pre && rows[s] >= 0) {
      const int64_t rowi = static_cast<int64_t>(bh) * v.row_capacity[s] + rows[s];
      vw[s] = *reinterpret_cast<const uint4*>(v.value_codes[s] + rowi * kCodeStride + 16 * quarter);
      vm[s] = *reinterpret_cast<const float2*>(v.value_meta[s] + (rowi * 2 + (quarter >> 1)) * 2);
    }
  }
  const uint16_t* vrow1 = nullptr;  // loop-2 V row for the fused source aggregate
  if (is_bf16) {
    const uint16_t* vrow = (t == cur) ? a.vc + static_cast<int64_t>(bh) * kDim
                                      : a.tail_v + (static_cast<int64_t>(bh) * v.tail_capacity + (t - Tp)) * kDim;
    if (kSource)
      vrow1 = (t == cur) ? a.vc1 + static_cast<int64_t>(bh) * kDim
                         : a.tail_v1 + (static_cast<int64_t>(bh) * v.tail_capacity + (t - Tp)) * kDim;
#pragma unroll
    for (int k = 0; k < 4; ++k) vbf[k] = *reinterpret_cast<const uint4*>(vrow + 32 * quarter + 8 * k);
  }

  // ---- logits of the selected keys
  float M = 0.0f;
  if (kSoftmax) {
    float d = 0.0f;
    if (is_bf16) {
      const uint16_t* krow =
          (t == cur) ? a.kc + static_cast<int64_t>(bh) * kDim
                     : a.tail_k + (static_cast<int64_t>(bh) * v.tail_capacity + (t - Tp)) * kDim;
#pragma unroll
      for (int k = 0; k < 4; ++k)
        d += dot_bf16_words(*reinterpret_cast<const uint4*>(krow + 32 * quarter + 8 * k), &qf[32 * quarter + 8 * k]);
    }
    for (int w0 = 0; w0 < nr; w0 += kWin) {
      // stage q*scale / q.min of runs [w0, w0+kWin): wave w owns runs w, w+kWaves, ...
      // and all their streams (stream index known at compile time, so the metadata
      // pointers stay in scalar registers)
      if (w0 > 0) load_meta(w0);
      const int nw = min(kWin, nr - w0);
      const float q0 = qf[2 * lane], q1 = qf[2 * lane + 1];
#pragma unroll
      for (int j = 0; j < kRunsPerWave; ++j) {
        const int wr = wave + kWaves * j;
        if (wr < nw) {  // wave-uniform
#pragma unroll
          for (int s = 0; s < NS; ++s) {
            qsh[wr][s][2 * lane] = q0 * meta[j][s].x;
            qsh[wr][s][2 * lane + 1] = q1 * meta[j][s].z * 0.0625f;  // high nibbles read as 16*code
            const float c = wave_sum(fmaf(q0, meta[j][s].y, q1 * meta[j][s].w));
            if (lane == 0) csh[wr][s] = c;
          }
        }
      }
      lds_barrier();
      if (is_pre && run >= w0 && run < w0 + kWin) {
        const int wr = run - w0;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          if (rows[s] < 0) continue;
          float qe[16], qo[16];
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const float4 x = *reinterpret_cast<const float4*>(&qsh[wr][s][32 * quarter + 8 * k]);
            const float4 y = *reinterpret_cast<const float4*>(&qsh[wr][s][32 * quarter + 8 * k + 4]);
            qe[4 * k + 0] = x.x; qo[4 * k + 0] = x.y;
            qe[4 * k + 1] = x.z; qo[4 * k + 1] = x.w;
            qe[4 * k + 2] = y.x; qo[4 * k + 2] = y.y;
            qe[4 * k + 3] = y.z; qo[4 * k + 3] = y.w;
          }
          float e = 0.0f;
          e = dot8(kw[s].x, qe + 0, qo + 0, e);
          e = dot8(kw[s].y, qe + 4, qo + 4, e);
          e = dot8(kw[s].z, qe + 8, qo + 8, e);
          e = dot8(kw[s].w, qe + 12, qo + 12, e);
          d += e;
          if (quarter == 0) d += csh[wr][s];
        }
      }
      lds_barrier();
    }
    d = quad_sum(d);
    const float lg = (t >= 0) ? d : -INFINITY;
    if (quarter == 0) pw[quad] = lg;
    lds_barrier();
    const float mt = wave_max(tid < kSlots ? pw[tid] : -INFINITY);
    if (lane == 0) msh[wave] = mt;
    lds_barrier();
    M = fmaxf(fmaxf(msh[0], msh[1]), fmaxf(msh[2], msh[3]));
    if (tid < kSlots) {
      const float l = pw[tid];
      pw[tid] = (l == -INFINITY) ? 0.0f : fast_exp2((l - M) * kLog2e);
    }
    lds_barrier();
  }

  // ---- P.V (and the fused loop-2 aggregate sum_S w V_1)
  const float p = pw[quad];
  const float w1 = kSource ? sw[quad] : 0.0f;
  float acc[32], acc1[kSource ? 32 : 1];
  float mu = 0.0f, mu1 = 0.0f;
#pragma unroll
  for (int c = 0; c < 32; ++c) acc[c] = 0.0f;
  if (kSource) {
#pragma unroll
    for (int c = 0; c < 32; ++c) acc1[c] = 0.0f;
  }
  if (is_pre) {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      if (rows[s] < 0) continue;
      const float we = p * vm[s].x;
      mu = fmaf(p, vm[s].y, mu);
      axpy8(vw[s].x, we, we * 0.0625f, acc + 0);
      axpy8(vw[s].y, we, we * 0.0625f, acc + 8);
      axpy8(vw[s].z, we, we * 0.0625f, acc + 16);
      axpy8(vw[s].w, we, we * 0.0625f, acc + 24);
      if (kSource && s < 2) {
        const float ws1 = w1 * vm[s].x;
        mu1 = fmaf(w1, vm[s].y, mu1);
        axpy8(vw[s].x, ws1, ws1 * 0.0625f, acc1 + 0);
        axpy8(vw[s].y, ws1, ws1 * 0.0625f, acc1 + 8);
        axpy8(vw[s].z, ws1, ws1 * 0.0625f, acc1 + 16);
        axpy8(vw[s].w, ws1, ws1 * 0.0625f, acc1 + 24);
      }
    }
  } else if (is_bf16) {
#pragma unroll
    for (int k = 0; k < 4; ++k) axpy_bf16_words(vbf[k], p, acc + 8 * k);
    if (kSource) {
#pragma unroll
      for (int k = 0; k < 4; ++k)
        axpy_bf16_words(*reinterpret_cast<const uint4*>(vrow1 + 32 * quarter + 8 * k), w1, acc1 + 8 * k);
    }
  }

  // ---- workgroup partial(s), then the last workgroup of the row merges it
  const int row = lane >> 2;
  float* part = a.ws + (static_cast<int64_t>(bh) * a.nchunk + chunk) * kPartial;
#pragma unroll
  for (int c = 0; c < 32; ++c) comb[wave][row][32 * quarter + c] = acc[c] + mu;
  if (quarter == 0) lsh[wave * 16 + row] = p;
  lds_barrier();
  if (tid < kDim) {
    float s = 0.0f;
    for (int w = 0; w < kWaves; ++w)
      for (int r = 0; r < 16; ++r) s += comb[w][r][tid];
    part[2 + tid] = s;
  } else if (tid == kDim) {
    float s = 0.0f;
    for (int i = 0; i < kWaves * 16; ++i) s += lsh[i];
    part[0] = (kSoftmax && s == 0.0f) ? -INFINITY : M;
    part[1] = s;
  }
  if (kSource) {
    lds_barrier();
    float* part1 = a.ws + (static_cast<int64_t>(gridDim.y) * a.nchunk + static_cast<int64_t>(bh) * a.nchunk + chunk) * kPartial;
#pragma unroll
    for (int c = 0; c < 32; ++c) comb[wave][row][32 * quarter + c] = acc1[c] + mu1;
    lds_barrier();
    if (tid < kDim) {
      float s = 0.0f;
      for (int w = 0; w < kWaves; ++w)
        for (int r = 0; r < 16; ++r) s += comb[w][r][tid];
      part1[2 + tid] = s;
    }
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
  FL_REQUIRE((capacity + kSlots - 1) / kSlots <= kMergeMaxParts, std::string(who) + ": capacity too large");
  FL_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 16 == 0, std::string(who) + ": workspace must be 16-byte aligned");
  return FL_OK;
}

size_t gather_workspace(int rows, int capacity, int sets) {
  const int nchunk = (capacity + kSlots - 1) / kSlots;
  return static_cast<size_t>(rows) * nchunk * kPartial * sizeof(float) * sets;
}

template <int MODE>
void launch_gather(GatherArgs& a, int rows, hipStream_t st) {
  const dim3 grid(a.nchunk, rows);
  a.tail_k = a.v.tail_key[a.loop];
  a.tail_v = a.v.tail_value[a.loop];
  a.tail_v1 = a.v.tail_value[1];
  switch (a.loop) {
    case 0: hipLaunchKernelGGL((gather_reader_kernel<1, MODE>), grid, dim3(kThreads), 0, st, a); break;
    case 1: hipLaunchKernelGGL((gather_reader_kernel<2, MODE>), grid, dim3(kThreads), 0, st, a); break;
    case 2: hipLaunchKernelGGL((gather_reader_kernel<3, MODE>), grid, dim3(kThreads), 0, st, a); break;
    default: hipLaunchKernelGGL((gather_reader_kernel<4, MODE>), grid, dim3(kThreads), 0, st, a); break;
  }
  const int mode = MODE == kSelectedPV ? kMergeSum : (MODE == kSparseDelta ? kMergeMassDelta : kMergeMassDeltaFused);
  const float* ws2 = a.ws + static_cast<int64_t>(rows) * a.nchunk * kPartial;
  hipLaunchKernelGGL(merge_partials_kernel, dim3(rows), dim3(kMergeThreads), 0, st, static_cast<const float*>(a.ws), a.nchunk,
                     a.out, mode, a.mass, a.src, ws2, a.src_out);
}

}  // namespace
}  // namespace fl

extern "C" size_t fl_decode_selected_workspace(const fl_cache_view* view, int32_t capacity) {
  using namespace fl;
  if (!view || capacity <= 0) return 0;
  // room for the fused variant's second partial set
  return gather_workspace(view->batch * view->heads, capacity, 2);
}

namespace {
float* gather_partials(void* workspace, int rows) {
  (void)rows;
  return static_cast<float*>(workspace);
}
}  // namespace

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
  const int rows = view->batch * view->heads;
  GatherArgs a{};
  a.v = *view;
  a.loop = loop;
  a.vc = v_cur;
  a.idx = indices;
  a.valid = valid;
  a.weights = weights;
  a.cap = capacity;
  a.ws = gather_partials(workspace, rows);
  a.nchunk = (capacity + kSlots - 1) / kSlots;
  a.out = out;
  launch_gather<kSelectedPV>(a, rows, static_cast<hipStream_t>(stream));
  FL_LAUNCH_CHECK("fl_decode_selected_pv");
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
  const int rows = view->batch * view->heads;
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
  a.ws = gather_partials(workspace, rows);
  a.nchunk = (capacity + kSlots - 1) / kSlots;
  a.out = out;
  a.mass = mass;
  a.src = source_output;
  launch_gather<kSparseDelta>(a, rows, static_cast<hipStream_t>(stream));
  FL_LAUNCH_CHECK("fl_decode_attn_sparse_delta");
  return FL_OK;
}

extern "C" int32_t fl_decode_attn_sparse_delta_fused(const fl_cache_view* view, int32_t loop, const uint16_t* q,
                                                     const uint16_t* k_cur, const uint16_t* v_cur,
                                                     const int32_t* indices, const uint8_t* valid,
                                                     const float* source_weights, const uint16_t* source_v_cur,
                                                     int32_t capacity, const float* mass, float scaling,
                                                     float* source_output, float* out, void* workspace,
                                                     size_t workspace_bytes, void* stream) {
  using namespace fl;
  clear_error();
  const int32_t rc = check_gather_args(view, loop, indices, valid, capacity, workspace, workspace_bytes,
                                       fl_decode_selected_workspace(view, capacity),
                                       "fl_decode_attn_sparse_delta_fused");
  if (rc != FL_OK) return rc;
  FL_REQUIRE(loop >= 2, "fl_decode_attn_sparse_delta_fused: loop must be 2 or 3");
  FL_REQUIRE(q && k_cur && v_cur && source_weights && source_v_cur && mass && source_output && out,
             "fl_decode_attn_sparse_delta_fused: null vector/output pointer");
  FL_REQUIRE(view->tail_value[1] != nullptr, "fl_decode_attn_sparse_delta_fused: null loop-2 tail");
  const int rows = view->batch * view->heads;
  GatherArgs a{};
  a.v = *view;
  a.loop = loop;
  a.q = q;
  a.kc = k_cur;
  a.vc = v_cur;
  a.idx = indices;
  a.valid = valid;
  a.weights = source_weights;
  a.vc1 = source_v_cur;
  a.cap = capacity;
  a.scaling = scaling;
  a.ws = gather_partials(workspace, rows);
  a.nchunk = (capacity + kSlots - 1) / kSlots;
  a.out = out;
  a.mass = mass;
  a.src_out = source_output;
  launch_gather<kSparseDeltaFused>(a, rows, static_cast<hipStream_t>(stream));
  FL_LAUNCH_CHECK("fl_decode_attn_sparse_delta_fused");
  return FL_OK;
}
