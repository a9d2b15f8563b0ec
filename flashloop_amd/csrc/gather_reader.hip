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
#include "reader_common.h"

#include <mutex>

namespace fl {
namespace {
using namespace reader;


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
  float* ws;              // partial slots [waves + B*H] (+ a second set for the fused source aggregate)
  int waves;              // persistent waves in the grid
  int tpr;                // tiles per row
  float* out;
  const float* mass;
  const float* src;       // source_output (kSparseDelta)
  float* src_out;         // source_output written (kSparseDeltaFused)
};

constexpr int kGatherSegs = 3;
constexpr int kLenCacheG = 512;  // batches whose lengths a reader caches in LDS  // row segments a wave stages before writing partials

__host__ __device__ __forceinline__ int64_t gather_slot(int w, int bh) { return static_cast<int64_t>(w) + bh; }

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

// ---------------------------------------------------------------------------------
// Persistent tile readers.  The selection of row bh is cut into tiles of T slots; wave
// w of the grid owns tiles [w*chunk, min((w+1)*chunk, total)) of the row-major tile
// sequence (chunk = ceil(total / waves)) and runs them one after another: a tile issues
// all its loads at once (index, then rank rows / codes / metadata) and many resident
// waves per CU overlap each other's load latencies.  Inside a tile LPT lanes own one
// slot (lane = LPT*n + part, 128/LPT channels per lane, T = 64/LPT slots).
//
// K metadata is per 64-token group: the tile stages q*scale (per channel) and q.min
// (per part) of W consecutive groups starting at its first prefix token's group in
// wave-private LDS; tokens beyond the window are handled by further windows.  It is
// read from the fp16 copy (key_meta_half): with ~6 selected tokens per group, the K
// metadata is half of these readers' bytes, and fp16 adds less error than the bf16
// rounding of the reference's residual chain that the fp32 stream sum already departs
// from.
// ---------------------------------------------------------------------------------
template <int LPT>
struct Lay {
  static constexpr int kTok = kWave / LPT;       // slots per tile
  static constexpr int kCh = kDim / LPT;         // channels per lane
  static constexpr int kWords = kRowBytes / LPT / 4;  // code words per lane
  static constexpr int kWin = LPT == 4 ? 4 : 2;  // K metadata window (groups)
};

template <int NS, int LPT>
struct TileLds {
  float qs[Lay<LPT>::kWin][NS][kDim];  // q*scale (odd channels pre-divided by 16)
  float qm[Lay<LPT>::kWin][NS][LPT];   // q.min per part
  float qf[kDim];                      // q*scaling of the current row
};

// Sum over the LPT lanes of a slot.
template <int LPT>
__device__ __forceinline__ float slot_sum(float x) {
  x += dpp<kDppXor1>(x);
  x += dpp<kDppXor2>(x);
  if (LPT == 8) x += dpp<kDppHalfMirror>(x);
  return x;
}

// Sum over the slots of a wave of values held per (slot, part): every lane gets the sum
// over the lanes with its part.
template <int LPT>
__device__ __forceinline__ float slots_sum(float x) {
  if (LPT == 4) x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x124, 0xF, 0xF, false));  // row_ror:4
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xF, 0xF, false));  // row_ror:8
  x += __shfl_xor(x, 16, kWave);
  x += __shfl_xor(x, 32, kWave);
  return x;
}

template <int LPT, int MODE>
struct TileOut {
  float m, l, mu, mu1;
  float acc[Lay<LPT>::kCh];
  float acc1[MODE == kSparseDeltaFused ? Lay<LPT>::kCh : 1];
};

template <int LPT, int MODE>
__device__ __forceinline__ void tile_reset(TileOut<LPT, MODE>& o) {
  o.m = (MODE == kSelectedPV) ? 0.0f : -INFINITY;
  o.l = o.mu = o.mu1 = 0.0f;
#pragma unroll
  for (int c = 0; c < Lay<LPT>::kCh; ++c) o.acc[c] = 0.0f;
  if (MODE == kSparseDeltaFused) {
#pragma unroll
    for (int c = 0; c < Lay<LPT>::kCh; ++c) o.acc1[c] = 0.0f;
  }
}

// Partial (m, l, acc[128]) of a wave segment -> staging LDS (second set: acc1 sums).
template <int LPT, int MODE>
__device__ __forceinline__ void tile_stage(const TileOut<LPT, MODE>& o, float* p, float* p1) {
  constexpr int kCh = Lay<LPT>::kCh;
  const int lane = threadIdx.x & 63, part = lane % LPT, n = lane / LPT;
  const float l = wave_sum(part == 0 ? o.l : 0.0f);
#pragma unroll
  for (int c = 0; c < kCh; ++c) {
    const float x = slots_sum<LPT>(o.acc[c] + o.mu);
    if (n == 0) p[2 + kCh * part + c] = x;
  }
  if (lane == 0) {
    p[0] = o.m;
    p[1] = l;
  }
  if (MODE == kSparseDeltaFused) {
#pragma unroll
    for (int c = 0; c < kCh; ++c) {
      const float x = slots_sum<LPT>(o.acc1[c] + o.mu1);
      if (n == 0) p1[2 + kCh * part + c] = x;
    }
    if (lane == 0) {
      p1[0] = 0.0f;
      p1[1] = 0.0f;
    }
  }
}

template <int LPT>
__device__ __forceinline__ void load_words(uint32_t* w, const uint8_t* src) {
  if (LPT == 4) {
    const uint4 x = *reinterpret_cast<const uint4*>(src);
    w[0] = x.x; w[1] = x.y; w[2] = x.z; w[3] = x.w;
  } else {
    const uint2 x = *reinterpret_cast<const uint2*>(src);
    w[0] = x.x; w[1] = x.y;
  }
}

__device__ __forceinline__ void wave_sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int NS, int MODE, int LPT>
__global__ __launch_bounds__(kThreads) void gather_reader_kernel(GatherArgs a) {
  using Y = Lay<LPT>;
  constexpr int kCh = Y::kCh, kWords = Y::kWords, kWin = Y::kWin;
  constexpr bool kSoftmax = MODE != kSelectedPV;
  constexpr bool kSource = MODE == kSparseDeltaFused;
  constexpr int kSets = kSource ? 2 : 1;
  __shared__ TileLds<NS, LPT> lds[kWaves];
  __shared__ float stage[kWaves][kGatherSegs][kSets][kPartial];
  __shared__ int seg_bh[kWaves][kGatherSegs];
  const fl_cache_view& v = a.v;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, part = lane % LPT, n = lane / LPT;
  const int half = part / (LPT / 2);
  const int w = blockIdx.x * kWaves + wave;
  TileLds<NS, LPT>& L = lds[wave];
  const int rows = v.batch * v.heads;
  const int tpr = a.cap / Y::kTok;  // tiles per row
  const int64_t total = static_cast<int64_t>(rows) * tpr;
  const int64_t chunk = (total + a.waves - 1) / a.waves;
  const int64_t t0 = static_cast<int64_t>(w) * chunk;
  const int64_t t1 = min(t0 + chunk, total);
  const int gcap = v.token_capacity / kGroup;

  auto write_stage = [&](int nseg) {
    wave_sync_lds();
    for (int k = 0; k < nseg; ++k) {
      const int sb = seg_bh[wave][k];
      for (int set = 0; set < kSets; ++set) {
        float* dst = a.ws + (static_cast<int64_t>(set) * (a.waves + rows) + gather_slot(w, sb)) * kPartial;
        for (int e = lane; e < kPartial; e += kWave) dst[e] = stage[wave][k][set][e];
      }
    }
  };

  // per-batch prefix length and current-token index, cached so the slot resolution of a
  // tile needs no length load
  __shared__ int len_tp[kLenCacheG], len_cur[kLenCacheG];
  for (int i = threadIdx.x; i < min(v.batch, kLenCacheG); i += kThreads) {
    // lengths come from device memory: clamp them to the buffers so a bad value cannot fault
    const int tp = min(max(v.packed_tokens[i], 0), v.token_capacity) & ~(kGroup - 1);
    len_tp[i] = tp;
    len_cur[i] = tp + min(max(v.tail_tokens[i], 0), v.tail_capacity);
  }
  __syncthreads();

  // Slot of this lane in a tile: token, stream rows, flags.  The index of tile j+1 is
  // loaded and its rank rows requested while tile j's codes are in flight and computed.
  struct Slot {
    int bh, b, Tp, cur, t;
    uint32_t has;
    int row[NS];
    float wt;
  };
  auto load_idx = [&](int64_t tile, int& ti, int& okv, float& wt) {
    const int bh = static_cast<int>(tile / tpr);
    const int64_t sel = static_cast<int64_t>(bh) * a.cap + (tile - static_cast<int64_t>(bh) * tpr) * Y::kTok + n;
    ti = a.idx[sel];
    okv = a.valid[sel];
    wt = (MODE != kSparseDelta) ? a.weights[sel] : 0.0f;
  };
  auto resolve = [&](int64_t tile, int ti, int okv, float wt) {
    Slot sl;
    sl.bh = static_cast<int>(tile / tpr);
    sl.b = sl.bh / v.heads;
    sl.Tp = sl.b < kLenCacheG ? len_tp[sl.b] : (min(max(v.packed_tokens[sl.b], 0), v.token_capacity) & ~(kGroup - 1));
    sl.cur = sl.b < kLenCacheG ? len_cur[sl.b] : sl.Tp + min(max(v.tail_tokens[sl.b], 0), v.tail_capacity);
    sl.t = (okv != 0 && ti >= 0 && ti <= sl.cur) ? ti : -1;  // out-of-range indices are dropped, never read
    sl.wt = wt;
    const bool pre = sl.t >= 0 && sl.t < sl.Tp;
    sl.has = 0;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      int r = pre ? sl.t : -1;
      if (s >= 2 && pre) {
        r = v.rank[s - 2][static_cast<int64_t>(sl.b) * v.token_capacity + sl.t];
        if (r >= v.row_capacity[s]) r = -1;
      }
      if (r >= 0) sl.has |= 1u << s;
      sl.row[s] = max(r, 0);
    }
    return sl;
  };

  TileOut<LPT, MODE> o;
  tile_reset<LPT, MODE>(o);
  int cur_bh = -1, nseg = 0;
  if (t0 >= t1) {
    write_stage(0);
    return;
  }
  int ti_n, ok_n;
  float wt_n;
  load_idx(t0, ti_n, ok_n, wt_n);
  Slot sl = resolve(t0, ti_n, ok_n, wt_n);

  for (int64_t tile = t0; tile < t1; ++tile) {
    const int64_t nxt = min(tile + 1, t1 - 1);  // the last tile re-reads its own index
    load_idx(nxt, ti_n, ok_n, wt_n);
    const int bh = sl.bh;
    if (bh != cur_bh) {
      if (cur_bh >= 0) {
        if (nseg == kGatherSegs) {  // stage full: write it out (rare)
          write_stage(nseg);
          nseg = 0;
        }
        tile_stage<LPT, MODE>(o, stage[wave][nseg][0], kSource ? stage[wave][nseg][kSets - 1] : nullptr);
        if (lane == 0) seg_bh[wave][nseg] = cur_bh;
        ++nseg;
        tile_reset<LPT, MODE>(o);
      }
      cur_bh = bh;
      if (kSoftmax) {
        wave_sync_lds();
        const uint32_t qw = *reinterpret_cast<const uint32_t*>(a.q + static_cast<int64_t>(bh) * kDim + 2 * lane);
        L.qf[2 * lane] = bf16lo_to_f32(qw) * a.scaling;
        L.qf[2 * lane + 1] = bf16hi_to_f32(qw) * a.scaling;
      }
    }
    const int t = sl.t, Tp = sl.Tp, cur = sl.cur;
    const uint32_t has = sl.has;
    const float wt = sl.wt;
    const bool pre = t >= 0 && t < Tp;
    const bool bf = t >= Tp;  // BF16 tail row or the current token
    // codes and V metadata of every stream (rows clamped: absent rows read row 0, masked below)
    uint32_t kw[NS][kWords], vw[NS][kWords];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const uint8_t* line = v.key_codes[s] + (static_cast<int64_t>(bh) * v.row_capacity[s] + sl.row[s]) * kCodeStride;
      if (kSoftmax) load_words<LPT>(kw[s], line + 4 * kWords * part);
      load_words<LPT>(vw[s], v.value_codes[s] - v.key_codes[s] + line + 4 * kWords * part);
    }
    // V metadata of every stream from the token's 64-byte record (this lane's half: 32 bytes)
    float2 vm[NS];
    {
      const float* rec = v.value_meta_token + ((static_cast<int64_t>(bh) * v.token_capacity + (pre ? t : 0)) * 2 + half) * 8;
      const float4 r01 = *reinterpret_cast<const float4*>(rec);
      const float4 r23 = NS > 2 ? *reinterpret_cast<const float4*>(rec + 4) : make_float4(0.f, 0.f, 0.f, 0.f);
      const float2 all[4] = {make_float2(r01.x, r01.y), make_float2(r01.z, r01.w), make_float2(r23.x, r23.y),
                             make_float2(r23.z, r23.w)};
#pragma unroll
      for (int s = 0; s < NS; ++s) vm[s] = all[s];
    }
    // first K-metadata window: groups from the first prefix token's (slots are sorted)
    const uint64_t pre_lanes = kSoftmax ? __ballot(pre) : 0;
    int gwin = 0;
    uint2 km[kSoftmax ? kWin : 1][NS];  // fp16 (scale, min) of channels 2*lane, 2*lane+1
    if (kSoftmax) {
      const int first = pre_lanes ? __builtin_ctzll(pre_lanes) : 0;
      const int tfirst = __shfl(t, first, kWave);
      gwin = pre_lanes ? tfirst / kGroup : 0;
#pragma unroll
      for (int j = 0; j < kWin; ++j)
#pragma unroll
        for (int s = 0; s < NS; ++s)
          km[j][s] = *reinterpret_cast<const uint2*>(
              v.key_meta_half[s] + ((static_cast<int64_t>(bh) * gcap + min(gwin + j, gcap - 1)) * kDim + 2 * lane) * 2);
    }
    // next tile's slot (rank rows fly while this tile computes)
    sl = resolve(nxt, ti_n, ok_n, wt_n);

    // ---- logits
    float lg = 0.0f;
    if (kSoftmax) {
      const int gtok = pre ? t / kGroup : -1;
      float d = 0.0f;
      for (bool first_win = true;; first_win = false) {  // windows of kWin groups (wave-uniform)
        if (!first_win) {
#pragma unroll
          for (int j = 0; j < kWin; ++j)
#pragma unroll
            for (int s = 0; s < NS; ++s)
              km[j][s] = *reinterpret_cast<const uint2*>(
                  v.key_meta_half[s] + ((static_cast<int64_t>(bh) * gcap + min(gwin + j, gcap - 1)) * kDim + 2 * lane) * 2);
        }
        const float q0 = L.qf[2 * lane], q1 = L.qf[2 * lane + 1];
        wave_sync_lds();  // earlier reads of the window buffers are done
#pragma unroll
        for (int j = 0; j < kWin; ++j)
#pragma unroll
          for (int s = 0; s < NS; ++s) {
            const float sc0 = f16_to_f32(km[j][s].x & 0xFFFFu), mn0 = f16_to_f32(km[j][s].x >> 16);
            const float sc1 = f16_to_f32(km[j][s].y & 0xFFFFu), mn1 = f16_to_f32(km[j][s].y >> 16);
            L.qs[j][s][2 * lane] = q0 * sc0;
            L.qs[j][s][2 * lane + 1] = q1 * sc1 * 0.0625f;  // high nibbles read as 16*code
            // q.min over the channels of one part: fold the kCh/2 lanes holding them
            float m = fmaf(q0, mn0, q1 * mn1);
            m += dpp<kDppXor1>(m);
            m += dpp<kDppXor2>(m);
            m += dpp<kDppHalfMirror>(m);
            if (LPT == 4) m += dpp<kDppMirror>(m);
            if ((lane & (kCh / 2 - 1)) == 0) L.qm[j][s][lane / (kCh / 2)] = m;
          }
        wave_sync_lds();
        const int js = gtok - gwin;
        if (pre && js >= 0 && js < kWin) {
#pragma unroll
          for (int s = 0; s < NS; ++s) {
            if (!((has >> s) & 1u)) continue;
            const float* qq = &L.qs[js][s][kCh * part];
            float e = 0.0f;
#pragma unroll
            for (int k = 0; k < kWords; ++k) {
              const float4 x = *reinterpret_cast<const float4*>(qq + 8 * k);
              const float4 y = *reinterpret_cast<const float4*>(qq + 8 * k + 4);
              const float qe[4] = {x.x, x.z, y.x, y.z}, qo[4] = {x.y, x.w, y.y, y.w};
              e = dot8(kw[s][k], qe, qo, e);
            }
            d += e + L.qm[js][s][part];
          }
        }
        // tokens past this window: another window
        const uint64_t rest = __ballot(pre && js >= kWin);
        if (!rest) break;
        gwin = __shfl(t, __builtin_ctzll(rest), kWave) / kGroup;
      }
      // BF16 tail rows and the current token
      if (__ballot(bf)) {
        if (bf) {
          const uint16_t* krow = (t == cur) ? a.kc + static_cast<int64_t>(bh) * kDim
                                            : a.tail_k + (static_cast<int64_t>(bh) * v.tail_capacity + (t - Tp)) * kDim;
#pragma unroll
          for (int k = 0; k < kCh / 8; ++k)
            d += dot_bf16_words(*reinterpret_cast<const uint4*>(krow + kCh * part + 8 * k), &L.qf[kCh * part + 8 * k]);
        }
      }
      d = slot_sum<LPT>(d);
      lg = t >= 0 ? d : -INFINITY;
      // online softmax over the wave's slots (m wave-uniform, rescaled lazily)
      const float tmax = wave_max(lg);
      if (tmax > o.m + 8.0f) {
        const float alpha = o.m == -INFINITY ? 0.0f : fast_exp2((o.m - tmax) * kLog2e);
        o.l *= alpha;
        o.mu *= alpha;
#pragma unroll
        for (int c = 0; c < kCh; ++c) o.acc[c] *= alpha;
        o.m = tmax;
      }
    }
    const float p = kSoftmax ? (t >= 0 ? fast_exp2((lg - o.m) * kLog2e) : 0.0f) : (t >= 0 ? wt : 0.0f);
    const float w1 = kSource ? (t >= 0 ? wt : 0.0f) : 0.0f;
    o.l += p;

    // ---- P.V (and the fused loop-2 aggregate sum_S w V_1)
    if (pre) {
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        if (!((has >> s) & 1u)) continue;
        const float we = p * vm[s].x;
        o.mu = fmaf(p, vm[s].y, o.mu);
#pragma unroll
        for (int k = 0; k < kWords; ++k) axpy8(vw[s][k], we, we * 0.0625f, o.acc + 8 * k);
        if (kSource && s < 2) {
          const float ws1 = w1 * vm[s].x;
          o.mu1 = fmaf(w1, vm[s].y, o.mu1);
#pragma unroll
          for (int k = 0; k < kWords; ++k) axpy8(vw[s][k], ws1, ws1 * 0.0625f, o.acc1 + 8 * k);
        }
      }
    }
    if (__ballot(bf)) {
      if (bf) {
        const uint16_t* vrow = (t == cur) ? a.vc + static_cast<int64_t>(bh) * kDim
                                          : a.tail_v + (static_cast<int64_t>(bh) * v.tail_capacity + (t - Tp)) * kDim;
#pragma unroll
        for (int k = 0; k < kCh / 8; ++k)
          axpy_bf16_words(*reinterpret_cast<const uint4*>(vrow + kCh * part + 8 * k), p, o.acc + 8 * k);
        if (kSource) {
          const uint16_t* vrow1 = (t == cur) ? a.vc1 + static_cast<int64_t>(bh) * kDim
                                             : a.tail_v1 + (static_cast<int64_t>(bh) * v.tail_capacity + (t - Tp)) * kDim;
#pragma unroll
          for (int k = 0; k < kCh / 8; ++k)
            axpy_bf16_words(*reinterpret_cast<const uint4*>(vrow1 + kCh * part + 8 * k), w1, o.acc1 + 8 * k);
        }
      }
    }
  }
  if (cur_bh >= 0) {
    if (nseg == kGatherSegs) {
      write_stage(nseg);
      nseg = 0;
    }
    tile_stage<LPT, MODE>(o, stage[wave][nseg][0], kSource ? stage[wave][nseg][kSets - 1] : nullptr);
    if (lane == 0) seg_bh[wave][nseg] = cur_bh;
    ++nseg;
  }
  write_stage(nseg);
}

// Merge of row bh: slots [f+bh, l+bh] of each partial set (see gather_slot).
__global__ __launch_bounds__(kMergeThreads) void gather_merge_kernel(const float* ws, int waves, int tpr, int nrows,
                                                                     float* out, int mode, const float* mass,
                                                                     const float* src, float* src_out) {
  __shared__ MergeLdsBuf S;
  const int bh = blockIdx.x, tid = threadIdx.x;
  const int64_t total = static_cast<int64_t>(nrows) * tpr;
  const int64_t chunk = (total + waves - 1) / waves;
  const int64_t f = static_cast<int64_t>(bh) * tpr / chunk, l = (static_cast<int64_t>(bh + 1) * tpr - 1) / chunk;
  const int64_t o = static_cast<int64_t>(bh) * kDim + tid;
  const MergeParts P{ws + (f + bh) * kPartial, static_cast<int>(l - f + 1), nullptr};
  if (mode == kMergeSum) {
    const float r = merge_channel_sum<false>(P, nullptr, S.acc);
    if (tid < kDim) out[o] = r;
    return;
  }
  float res = merge_softmax(P, S);
  if (mode == kMergeMassDeltaFused) {
    const MergeParts P2{ws + (static_cast<int64_t>(waves) + nrows + f + bh) * kPartial, static_cast<int>(l - f + 1),
                        nullptr};
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

int32_t check_gather_args(const fl_cache_view* view, int32_t loop, const int32_t* indices, const uint8_t* valid,
                          int32_t capacity, void* workspace, size_t workspace_bytes, size_t need, const char* who) {
  FL_REQUIRE(view != nullptr, std::string(who) + ": view is null");
  const fl_cache_view& v = *view;
  FL_REQUIRE(loop >= 0 && loop <= 3, std::string(who) + ": loop must be in 0..3");
  FL_REQUIRE(indices && valid && workspace, std::string(who) + ": null indices/valid/workspace");
  FL_REQUIRE(capacity > 0 && capacity % 16 == 0, std::string(who) + ": capacity must be a positive multiple of 16");
  FL_REQUIRE(v.batch > 0 && v.heads > 0 && v.token_capacity % kGroup == 0, std::string(who) + ": bad view geometry");
  FL_REQUIRE(v.packed_tokens && v.tail_tokens, std::string(who) + ": null length arrays");
  FL_REQUIRE(v.tail_key[loop] && v.tail_value[loop], std::string(who) + ": null tail for this loop");
  for (int s = 0; s <= loop && v.max_packed_tokens > 0; ++s) {
    FL_REQUIRE(v.key_codes[s] && v.key_meta[s] && v.value_codes[s] && v.value_meta[s] && v.value_meta_token &&
                   v.key_meta_half[s],
               std::string(who) + ": null stream pointer");
    if (s >= 2) FL_REQUIRE(v.rank[s - 2] != nullptr, std::string(who) + ": null rank map");
  }
  FL_REQUIRE(workspace_bytes >= need, std::string(who) + ": workspace too small");
  FL_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 16 == 0, std::string(who) + ": workspace must be 16-byte aligned");
  return FL_OK;
}

int gather_cu_count() {
  static std::mutex mu;
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::lock_guard<std::mutex> g(mu);
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

template <int NS, int MODE, int LPT>
int gather_occupancy() {
  static std::mutex mu;
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 1;
  std::lock_guard<std::mutex> g(mu);
  if (cached[dev] == 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, gather_reader_kernel<NS, MODE, LPT>, kThreads, 0) != hipSuccess ||
        n <= 0)
      n = 1;
    cached[dev] = n;
  }
  return cached[dev];
}

constexpr int kGatherMaxResident = 4;  // workgroups per CU any reader instantiation holds

// Persistent grid: every resident workgroup slot, fewer when the selection is small.
int gather_blocks(int rows, int capacity, int occ) {
  const int64_t tiles = static_cast<int64_t>(rows) * (capacity / 16);  // upper bound over tile sizes
  const int64_t want = (tiles + kWaves - 1) / kWaves;
  const int64_t slots = static_cast<int64_t>(gather_cu_count()) * std::min(std::max(occ, 1), kGatherMaxResident);
  return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(slots, want)));
}

size_t gather_workspace(int rows, int capacity) {
  const int64_t waves = static_cast<int64_t>(gather_blocks(rows, capacity, kGatherMaxResident)) * kWaves;
  return static_cast<size_t>(2 * (waves + rows)) * kPartial * sizeof(float);
}

#ifndef FL_GATHER_LPT
#define FL_GATHER_LPT 8
#endif
constexpr int kLpt = FL_GATHER_LPT;  // lanes per selected slot

template <int NS, int MODE>
void launch_ns(GatherArgs& a, int rows, hipStream_t st) {
  const int blocks = gather_blocks(rows, a.cap, gather_occupancy<NS, MODE, kLpt>());
  a.waves = blocks * kWaves;
  a.tpr = a.cap / Lay<kLpt>::kTok;
  hipLaunchKernelGGL((gather_reader_kernel<NS, MODE, kLpt>), dim3(blocks), dim3(kThreads), 0, st, a);
}

template <int MODE>
void launch_gather(GatherArgs& a, int rows, hipStream_t st) {
  a.tail_k = a.v.tail_key[a.loop];
  a.tail_v = a.v.tail_value[a.loop];
  a.tail_v1 = a.v.tail_value[1];
  switch (a.loop) {
    case 0: launch_ns<1, MODE>(a, rows, st); break;
    case 1: launch_ns<2, MODE>(a, rows, st); break;
    case 2: launch_ns<3, MODE>(a, rows, st); break;
    default: launch_ns<4, MODE>(a, rows, st); break;
  }
  const int mode = MODE == kSelectedPV ? kMergeSum : (MODE == kSparseDelta ? kMergeMassDelta : kMergeMassDeltaFused);
  hipLaunchKernelGGL(gather_merge_kernel, dim3(rows), dim3(kMergeThreads), 0, st, static_cast<const float*>(a.ws),
                     a.waves, a.tpr, rows, a.out, mode, a.mass, a.src, a.src_out);
}

}  // namespace
}  // namespace fl

extern "C" size_t fl_decode_selected_workspace(const fl_cache_view* view, int32_t capacity) {
  using namespace fl;
  if (!view || capacity <= 0) return 0;
  // room for the fused variant's second partial set
  return gather_workspace(view->batch * view->heads, capacity);
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
  a.out = out;
  a.mass = mass;
  a.src_out = source_output;
  launch_gather<kSparseDeltaFused>(a, rows, static_cast<hipStream_t>(stream));
  FL_LAUNCH_CHECK("fl_decode_attn_sparse_delta_fused");
  return FL_OK;
}
