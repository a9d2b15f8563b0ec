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
  const int32_t* counts;  // selected slots per row (nullable: every row holds `cap`)
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

constexpr int kGatherSegs = 3;   // row segments a wave stages (its first one until the end)
constexpr int kLenCacheG = 512;  // batches whose lengths a reader caches in LDS
constexpr int kLiveRows = 2048;  // rows whose live-tile prefix a reader keeps in LDS

// ---------------------------------------------------------------------------------
// Live tiles.  With per-row selected counts, row r holds max(1, ceil(count_r / T)) live
// tiles (T slots per tile; count clamped to [0, cap]) and the readers partition only
// those, so a ragged batch's padding slots cost no wave time; without counts (or beyond
// kLiveRows rows) every row holds cap / T tiles.  A row keeps at least one tile, so a row
// with nothing selected still gets its (empty) partial.  The reader and the merge derive
// the same integers from the same counts.
// ---------------------------------------------------------------------------------
__device__ __forceinline__ int live_tiles(const int32_t* counts, int r, int cap, int tok) {
  const int c = min(max(counts[r], 0), cap);
  return max((c + tok - 1) / tok, 1);
}

__device__ __forceinline__ int wave_sum_int(int x) {
#pragma unroll
  for (int d = kWave / 2; d >= 1; d >>= 1) x += __shfl_xor(x, d, kWave);
  return x;
}

// pre[r] = live tiles of rows 0..r-1, r = 0..rows (kThreads threads; rows <= kLiveRows),
// in two halves so that a caller can issue other loads between them: live_load reads this
// thread's rows, live_prefix scans them (and ends with a barrier).
constexpr int kLivePer = (kLiveRows + kThreads - 1) / kThreads;
__device__ __forceinline__ void live_load(int* mine, const int32_t* counts, int rows, int cap, int tok) {
  const int r0 = threadIdx.x * kLivePer;
#pragma unroll
  for (int k = 0; k < kLivePer; ++k) mine[k] = r0 + k < rows ? live_tiles(counts, r0 + k, cap, tok) : 0;
}
__device__ __forceinline__ void live_prefix(int* pre, int* wave_tot, const int* mine, int rows) {
  constexpr int kPer = kLivePer;
  const int tid = threadIdx.x, lane = tid & 63;
  const int r0 = tid * kPer;
  int s = 0;
#pragma unroll
  for (int k = 0; k < kPer; ++k) s += mine[k];
  // inclusive scan over the wave, then the earlier waves' totals
  int x = s;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int y = __shfl_up(x, d, kWave);
    if (lane >= d) x += y;
  }
  if (lane == kWave - 1) wave_tot[tid >> 6] = x;
  __syncthreads();
  int base = x - s;
  for (int w = 0; w < (tid >> 6); ++w) base += wave_tot[w];
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    if (r0 + k < rows) pre[r0 + k] = base;
    base += mine[k];
  }
  if (tid == kThreads - 1) pre[rows] = base;  // the last thread's rows end the sequence
  __syncthreads();
}

// Partial slot of row bh from workgroup g: a workgroup's tile range is contiguous, so the
// slots of one row are contiguous and disjoint from every other row's.
__host__ __device__ __forceinline__ int64_t gather_slot(int g, int bh) { return static_cast<int64_t>(g) + bh; }

// A wave-uniform 64-bit value computed on the vector unit (e.g. a division) moved to
// scalar registers, so the values derived from it stay scalar too.
__device__ __forceinline__ int64_t uniform64(int64_t x) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(x));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(static_cast<uint64_t>(x) >> 32));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

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
// sequence (chunk = ceil(total / waves); the sequence holds only each row's live tiles
// when counts are given) and runs them one after another: a tile issues
// all its loads at once (index, then rank rows / codes / metadata) and many resident
// waves per CU overlap each other's load latencies.  Inside a tile LPT lanes own one
// slot (lane = LPT*n + part, 128/LPT channels per lane, T = 64/LPT slots).  The four
// waves of a workgroup own consecutive ranges; at the end they combine their (m, l, acc)
// of each row they share, so a row has one partial per workgroup that touched it (a
// quarter of the parts its merge reads at batch one, where every wave runs one tile).
//
// K metadata is per 64-token group.  A wave keeps q*scale (per channel) and q.min (per
// part) of the last kRing groups it loaded in a wave-private LDS ring; as its tiles walk
// a row's sorted selection, each tile loads only the groups past those already in the
// ring (about 1.3 per 8-slot tile at 10% retention, instead of a fixed window), so every
// group's metadata is fetched about once per row and stream.  Metadata is read from the
// fp16 copy (key_meta_half): with ~6 selected tokens per group, the K metadata is a large
// share of these readers' requests, and fp16 adds less error than the bf16 rounding of
// the reference's residual chain that the fp32 stream sum already departs from.
// ---------------------------------------------------------------------------------
template <int LPT>
struct Lay {
  static constexpr int kTok = kWave / LPT;       // slots per tile
  static constexpr int kCh = kDim / LPT;         // channels per lane
  static constexpr int kWords = kRowBytes / LPT / 4;  // code words per lane
};
constexpr int kRing = 4;  // K-metadata groups a wave keeps (q*scale form) in LDS
constexpr int kNew = 2;   // groups a tile may add to the ring

template <int NS, int LPT>
struct TileLds {
  uint32_t qs[kRing][NS][kDim / 2];  // fp16 q*scale*2^-E of group g in ring slot g % kRing (dot8h2 pairs)
  float qm[kRing][NS][LPT];          // q.min per part
  uint32_t qs1[NS][kDim / 2];        // one group for tiles that do not fit the ring
  float qm1[NS][LPT];
  float qf[kDim];             // q*scaling of the current row
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

// Load a T at byte offset `off` (32-bit, unsigned) of a wave-uniform base: compiles to a
// global load with a scalar base and one 32-bit offset register.
template <typename T>
__device__ __forceinline__ T load_at(const void* base, uint32_t off) {
  return *reinterpret_cast<const T*>(reinterpret_cast<const char*>(base) + off);
}

__device__ __forceinline__ void wave_sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The tile loop is a software pipeline three tiles deep, so that a wave always has the
// code loads of one tile in flight while it computes another:
//   iteration j issues the selection record of tile j+3, the rank rows of tile j+2 (from
//   the record loaded in iteration j-1) and the codes/metadata of tile j+1 (rows from
//   the rank loads of iteration j-1), then computes tile j.
// Every load of the steady state is unconditional (absent rows read a clamped row and
// are masked), so the compiler's in-order wait before tile j's arithmetic counts only
// the loads issued after tile j's.  The loop is unrolled by two with two register sets
// (a copy of a set still in flight would wait for its loads).
template <int NS, int MODE, int LPT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2))) void gather_reader_kernel(GatherArgs a) {
  using Y = Lay<LPT>;
  constexpr int kCh = Y::kCh, kWords = Y::kWords;
  constexpr bool kSoftmax = MODE != kSelectedPV;
  constexpr bool kSource = MODE == kSparseDeltaFused;
  constexpr int kSets = kSource ? 2 : 1;
  constexpr int kNR = NS > 2 ? NS - 2 : 1;  // rank maps read (streams 2, 3)
  __shared__ TileLds<NS, LPT> lds[kWaves];
  __shared__ float stage[kWaves][kGatherSegs][kSets][kPartial];
  __shared__ int seg_bh[kWaves][kGatherSegs];
  __shared__ int seg_n[kWaves];
  const fl_cache_view& v = a.v;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, part = lane % LPT, n = lane / LPT;
  const int half = part / (LPT / 2);
  // wave-uniform values live in scalar registers: every load below is a scalar base plus
  // a 32-bit lane offset
  const int w = blockIdx.x * kWaves + __builtin_amdgcn_readfirstlane(wave);
  TileLds<NS, LPT>& L = lds[wave];
  const int rows = v.batch * v.heads;
  const int tpr = a.cap / Y::kTok;  // tiles per row (without counts)
  __shared__ int live_pre[kLiveRows + 1];
  __shared__ int live_wt[kWaves];
  const bool by_count = a.counts != nullptr && rows <= kLiveRows;
  int live_mine[kLivePer];
  if (by_count) live_load(live_mine, a.counts, rows, a.cap, Y::kTok);  // in flight with the length loads below
  const int gcap = v.token_capacity / kGroup;

  // Segments k0..n-1 of this wave: rows that start and end inside the wave's range, so no
  // other wave has a partial of them (written straight to the workgroup's slot).
  auto write_stage = [&](int k0, int n) {
    wave_sync_lds();
    for (int k = k0; k < n; ++k) {
      const int sb = seg_bh[wave][k];
      for (int set = 0; set < kSets; ++set) {
        float* dst = a.ws + (static_cast<int64_t>(set) * (a.waves + rows) + gather_slot(blockIdx.x, sb)) * kPartial;
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
  if (by_count) live_prefix(live_pre, live_wt, live_mine, rows);  // (its barriers also order the length cache)
  else __syncthreads();
  const int64_t total = by_count ? static_cast<int64_t>(__builtin_amdgcn_readfirstlane(live_pre[rows]))
                                 : static_cast<int64_t>(rows) * tpr;
  const int64_t chunk = uniform64((total + a.waves - 1) / a.waves);
  const int64_t t0 = static_cast<int64_t>(w) * chunk;
  const int64_t t1 = min(t0 + chunk, total);

  // Tile cursor: row, batch, tile within the row.  Cursors advance one tile at a time (an
  // integer division per tile would cost ~100 scalar instructions) and stop at the last
  // tile (tiles past the end are loaded again, never computed).
  struct Pos {
    int64_t i;
    int bh, b, h, k, kend;  // kend: live tiles of row bh
  };
  auto pos_at = [&](int64_t tile) {
    Pos p;
    p.i = tile;
    if (by_count) {
      int lo = 0, hi = rows;  // live_pre[lo] <= tile < live_pre[hi]
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (live_pre[mid] <= tile) lo = mid;
        else hi = mid;
      }
      p.bh = __builtin_amdgcn_readfirstlane(lo);
      p.k = __builtin_amdgcn_readfirstlane(static_cast<int>(tile - live_pre[p.bh]));
      p.kend = __builtin_amdgcn_readfirstlane(live_pre[p.bh + 1] - live_pre[p.bh]);
    } else {
      p.bh = __builtin_amdgcn_readfirstlane(static_cast<int>(tile / tpr));
      p.k = __builtin_amdgcn_readfirstlane(static_cast<int>(tile - static_cast<int64_t>(p.bh) * tpr));
      p.kend = tpr;
    }
    p.b = __builtin_amdgcn_readfirstlane(p.bh / v.heads);
    p.h = p.bh - p.b * v.heads;
    return p;
  };
  auto step = [&](Pos& p) {
    if (p.i + 1 >= t1) return;
    ++p.i;
    if (++p.k == p.kend) {
      p.k = 0;
      ++p.bh;
      if (++p.h == v.heads) {
        p.h = 0;
        ++p.b;
      }
      if (by_count) p.kend = __builtin_amdgcn_readfirstlane(live_pre[p.bh + 1] - live_pre[p.bh]);
    }
  };

  // ---- stage 1: the selection record of this lane's slot
  struct Rec {
    int ti, ok;
    float wt;
  };
  auto load_rec = [&](const Pos& p) {
    const int64_t sel0 = static_cast<int64_t>(p.bh) * a.cap + p.k * Y::kTok;
    Rec r;
    r.ti = load_at<int>(a.idx + sel0, 4u * n);
    r.ok = load_at<uint8_t>(a.valid + sel0, static_cast<uint32_t>(n));
    r.wt = (MODE != kSparseDelta) ? load_at<float>(a.weights + sel0, 4u * n) : 0.0f;
    return r;
  };
  // ---- stage 2: the slot (token, lengths) and the raw rank rows of streams 2/3
  struct Slot {
    int bh, b, Tp, cur, t;
    float wt;
    int rr[kNR];
  };
  auto resolve = [&](const Pos& p, const Rec& r) {
    Slot sl;
    sl.bh = p.bh;
    sl.b = p.b;
    sl.Tp = sl.b < kLenCacheG ? len_tp[sl.b] : (min(max(v.packed_tokens[sl.b], 0), v.token_capacity) & ~(kGroup - 1));
    sl.cur = sl.b < kLenCacheG ? len_cur[sl.b] : sl.Tp + min(max(v.tail_tokens[sl.b], 0), v.tail_capacity);
    sl.t = (r.ok != 0 && r.ti >= 0 && r.ti <= sl.cur) ? r.ti : -1;  // out-of-range indices are dropped, never read
    sl.wt = r.wt;
    const bool pre = sl.t >= 0 && sl.t < sl.Tp;
#pragma unroll
    for (int s = 2; s < NS; ++s)  // unconditional (token 0 for non-prefix slots): masked in stage 3
      sl.rr[s - 2] = load_at<int>(v.rank[s - 2] + static_cast<int64_t>(sl.b) * v.token_capacity,
                                  4u * static_cast<uint32_t>(pre ? sl.t : 0));
    return sl;
  };
  // ---- stage 3: codes, V records, new K-metadata groups and query word of a tile
  struct Tile {
    int bh, t, Tp, cur;
    uint32_t has;
    float wt;
    int glo, nnew;       // groups glo .. glo+nnew-1 loaded into km (ring additions)
    int gfirst, glast;   // group span of the tile's prefix slots
    bool fits;           // every group of the span is in the ring after the additions
    uint32_t qw;
    uint32_t kw[NS][kWords], vw[NS][kWords];
    float4 vm01, vm23;
    uint2 km[kSoftmax ? kNew : 1][NS];  // fp16 (scale, min) of channels 2*lane, 2*lane+1
  };
  // groups already requested for the ring, in issue order (wave-uniform)
  int ld_bh = -1, ld_hi = -1;
  auto issue = [&](const Slot& sl) {
    Tile T;
    T.bh = sl.bh;
    T.t = sl.t;
    T.Tp = sl.Tp;
    T.cur = sl.cur;
    T.wt = sl.wt;
    const bool pre = sl.t >= 0 && sl.t < sl.Tp;
    T.has = 0;
    int row[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      int r = pre ? sl.t : -1;
      if (s >= 2 && pre) {
        r = sl.rr[s - 2];
        if (r >= v.row_capacity[s]) r = -1;
      }
      if (r >= 0) T.has |= 1u << s;
      row[s] = max(r, 0);
    }
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      // row base (scalar) + line offset (32-bit: row < row_capacity <= 2^24, checked on the host)
      const int64_t base = static_cast<int64_t>(sl.bh) * v.row_capacity[s] * kCodeStride;
      const uint32_t off = static_cast<uint32_t>(row[s]) * kCodeStride + 4 * kWords * part;
      if (kSoftmax) load_words<LPT>(T.kw[s], v.key_codes[s] + base + off);
      load_words<LPT>(T.vw[s], v.key_codes[s] + base + off + kCodeStride / 2);  // V row: second half of the line
    }
    // V metadata of every stream from the token's 64-byte record (this lane's half: 32 bytes)
    const float* rec = v.value_meta_token + static_cast<int64_t>(sl.bh) * v.token_capacity * 16;
    const uint32_t roff = static_cast<uint32_t>(pre ? sl.t : 0) * 64u + half * 32u;
    T.vm01 = load_at<float4>(rec, roff);
    T.vm23 = NS > 2 ? load_at<float4>(rec, roff + 16u) : make_float4(0.f, 0.f, 0.f, 0.f);
    T.glo = 0;
    T.nnew = 0;
    T.gfirst = 0;
    T.glast = -1;
    T.fits = true;
    if (kSoftmax) {
      // group span of the prefix slots (slots are sorted) and the groups new to the ring
      const uint64_t pre_lanes = __ballot(pre);
      if (pre_lanes) {
        T.gfirst = __builtin_amdgcn_readfirstlane(__shfl(sl.t, __builtin_ctzll(pre_lanes), kWave)) / kGroup;
        T.glast = __builtin_amdgcn_readfirstlane(__shfl(sl.t, 63 - __builtin_clzll(pre_lanes), kWave)) / kGroup;
      }
      T.glo = sl.bh == ld_bh ? max(T.gfirst, ld_hi + 1) : T.gfirst;
      const int want = T.glast - T.glo + 1;
      T.nnew = min(max(want, 0), kNew);
      T.fits = T.glast - T.gfirst < kRing && want <= kNew;
      if (T.nnew > 0) {
        ld_bh = sl.bh;
        ld_hi = T.glo + T.nnew - 1;
      }
#pragma unroll
      for (int j = 0; j < kNew; ++j)
        if (j < T.nnew)
#pragma unroll
          for (int s = 0; s < NS; ++s)
            T.km[j][s] = load_at<uint2>(v.key_meta_half[s] + (static_cast<int64_t>(sl.bh) * gcap + T.glo + j) * kDim * 2,
                                        8u * lane);
      T.qw = load_at<uint32_t>(a.q + static_cast<int64_t>(sl.bh) * kDim, 4u * lane);
    }
    return T;
  };

  TileOut<LPT, MODE> o;
  tile_reset<LPT, MODE>(o);
  int cur_bh = -1, nseg = 0;
  // the row's q*scaling is staged as fp16 factors q*scale*2^-E, with 2^E above max|q*scaling|
  // so that every factor is at most |scale| (a finite fp16 scale gives a finite factor)
  float qn = 1.0f, qe = kSub16;  // 2^-E and 2^(24+E)

  // ---- stage 4: the arithmetic of a tile
  auto compute = [&](Tile& T) {
    const int bh = T.bh;
    if (bh != cur_bh) {
      if (cur_bh >= 0) {
        if (nseg == kGatherSegs) {  // stage full (rare): write the whole rows out, keep the first
          write_stage(1, nseg);
          nseg = 1;
        }
        tile_stage<LPT, MODE>(o, stage[wave][nseg][0], kSource ? stage[wave][nseg][kSets - 1] : nullptr);
        if (lane == 0) seg_bh[wave][nseg] = cur_bh;
        ++nseg;
        tile_reset<LPT, MODE>(o);
      }
      cur_bh = bh;
      if (kSoftmax) {
        wave_sync_lds();
        const float f0 = bf16lo_to_f32(T.qw) * a.scaling, f1 = bf16hi_to_f32(T.qw) * a.scaling;
        L.qf[2 * lane] = f0;
        L.qf[2 * lane + 1] = f1;
        const float amax = wave_max(fmaxf(fabsf(f0), fabsf(f1)));
        int e = 0;
        if (amax > 0.0f && amax <= 3.0e38f) frexpf(amax, &e);
        e = min(max(e, -100), 100);
        qn = ldexpf(1.0f, -e);
        qe = ldexpf(kSub16, e);
      }
    }
    const int t = T.t, Tp = T.Tp, cur = T.cur;
    const uint32_t has = T.has;
    const bool pre = t >= 0 && t < Tp;
    const bool bf = t >= Tp;  // BF16 tail row or the current token
    float2 vm[NS];
    {
      const float2 all[4] = {make_float2(T.vm01.x, T.vm01.y), make_float2(T.vm01.z, T.vm01.w),
                             make_float2(T.vm23.x, T.vm23.y), make_float2(T.vm23.z, T.vm23.w)};
#pragma unroll
      for (int s = 0; s < NS; ++s) vm[s] = all[s];
    }

    // ---- logits
    float lg = 0.0f;
    if (kSoftmax) {
      const int gtok = pre ? t / kGroup : -1;
      const float q0 = L.qf[2 * lane], q1 = L.qf[2 * lane + 1];
      // fp16 (scale, min) of one group and stream -> q*scale (this lane's two channels) and
      // q.min (folded over the kCh/2 lanes of one part)
      auto stage_group = [&](uint2 km, uint32_t* qs, float* qm) {
        const float sc0 = f16_to_f32(km.x & 0xFFFFu), mn0 = f16_to_f32(km.x >> 16);
        const float sc1 = f16_to_f32(km.y & 0xFFFFu), mn1 = f16_to_f32(km.y >> 16);
        uint16_t* qh = reinterpret_cast<uint16_t*>(qs);
        const int at = pair_slot(2 * lane);  // channel 2*lane + 1 sits one pair later
        qh[at] = __builtin_bit_cast(uint16_t, static_cast<_Float16>((q0 * qn) * sc0));
        qh[at + 2] = __builtin_bit_cast(uint16_t, static_cast<_Float16>((q1 * (qn * 0.0625f)) * sc1));  // read as 16*code
        float m = fmaf(q0, mn0, q1 * mn1);
        m += dpp<kDppXor1>(m);
        m += dpp<kDppXor2>(m);
        m += dpp<kDppHalfMirror>(m);
        if (LPT == 4) m += dpp<kDppMirror>(m);
        if ((lane & (kCh / 2 - 1)) == 0) qm[lane / (kCh / 2)] = m;
      };
      // logit of this lane's slot from the staged q*scale / q.min of its group
      auto dot_group = [&](const uint32_t (*qs)[kDim / 2], const float (*qm)[LPT]) {
        float d = 0.0f;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          // streams 0/1 hold every prefix token; stream 2 is selected, not branched over
          // (an absent row reads row 0's codes, which the select discards); stream 3 is
          // branched over (selecting it too costs the loop-4 kernel registers it spills)
          if (s == 3 && !((has >> s) & 1u)) continue;
          const uint32_t* qq = &qs[s][kCh / 2 * part];
          float e = 0.0f;
#pragma unroll
          for (int k = 0; k < kWords; ++k) e = dot8h2(T.kw[s][k], *reinterpret_cast<const uint4*>(qq + 4 * k), e);
          const float t = fmaf(e, qe, qm[s][part]);
          d += (s != 2 || ((has >> s) & 1u)) ? t : 0.0f;
        }
        return d;
      };
      // the tile's new groups -> ring (their loads were issued with the tile)
      if (T.nnew > 0) {
        wave_sync_lds();  // earlier reads of the ring slots are done
#pragma unroll
        for (int j = 0; j < kNew; ++j)
          if (j < T.nnew) {
            const int r = (T.glo + j) & (kRing - 1);
#pragma unroll
            for (int s = 0; s < NS; ++s) stage_group(T.km[j][s], L.qs[r][s], L.qm[r][s]);
          }
        wave_sync_lds();
      }
      float d = 0.0f;
      if (T.fits) {
        if (pre) {
          const int r = gtok & (kRing - 1);
          d = dot_group(L.qs[r], L.qm[r]);
        }
      } else {
        // rare: the span exceeds the ring -- one group at a time, loaded on demand
        for (int g = T.gfirst; g <= T.glast; ++g) {
          if (!__ballot(pre && gtok == g)) continue;
          uint2 km1[NS];
#pragma unroll
          for (int s = 0; s < NS; ++s)
            km1[s] = load_at<uint2>(v.key_meta_half[s] + (static_cast<int64_t>(bh) * gcap + g) * kDim * 2, 8u * lane);
          wave_sync_lds();
#pragma unroll
          for (int s = 0; s < NS; ++s) stage_group(km1[s], L.qs1[s], L.qm1[s]);
          wave_sync_lds();
          if (pre && gtok == g) d = dot_group(L.qs1, L.qm1);
        }
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
      // online softmax over the wave's slots (m wave-uniform, rescaled lazily); the
      // wave's maximum is formed only when some slot exceeds m by more than e^8
      if (__ballot(lg > o.m + 8.0f)) {
        const float tmax = wave_max(lg);
        const float alpha = o.m == -INFINITY ? 0.0f : fast_exp2((o.m - tmax) * kLog2e);
        o.l *= alpha;
        o.mu *= alpha;
#pragma unroll
        for (int c = 0; c < kCh; ++c) o.acc[c] *= alpha;
        o.m = tmax;
      }
    }
    const float p = kSoftmax ? (t >= 0 ? fast_exp2((lg - o.m) * kLog2e) : 0.0f) : (t >= 0 ? T.wt : 0.0f);
    const float w1 = kSource ? (t >= 0 ? T.wt : 0.0f) : 0.0f;
    o.l += p;

    // ---- P.V (and the fused loop-2 aggregate sum_S w V_1)
    if (pre) {
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        // an absent stream-2 row (row 0's codes were read) gets weight 0 by a select;
        // stream 3 is branched over
        if (s == 3 && !((has >> s) & 1u)) continue;
        const bool in = s != 2 || ((has >> s) & 1u);
        const float we = in ? (p * kSub16) * vm[s].x : 0.0f;  // codes read as fp16 subnormals (axpy8h)
        o.mu += in ? p * vm[s].y : 0.0f;
#pragma unroll
        for (int k = 0; k < kWords; ++k) axpy8h(T.vw[s][k], we, we * 0.0625f, o.acc + 8 * k);
        if (kSource && s < 2) {
          const float ws1 = (w1 * kSub16) * vm[s].x;
          o.mu1 = fmaf(w1, vm[s].y, o.mu1);
#pragma unroll
          for (int k = 0; k < kWords; ++k) axpy8h(T.vw[s][k], ws1, ws1 * 0.0625f, o.acc1 + 8 * k);
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
  };

  // ---- prologue: tile t0 issued, rank rows of t0+1 and records of t0+2 in flight.  Each
  // iteration issues in age order record(j+3), rank(j+2), codes(j+1): a wait for one of
  // them never waits for younger code loads.
  if (t0 < t1) {
    Slot s_next;
    Rec r_next;
    Tile A, B;
    Pos pr = pos_at(t0);  // cursor of the next selection record to load
    Pos ps = pr;          // cursor of the next slot to resolve
    {
      const Rec r0 = load_rec(pr);
      step(pr);
      const Rec r1 = load_rec(pr);
      step(pr);
      r_next = load_rec(pr);
      const Slot s0 = resolve(ps, r0);
      step(ps);
      s_next = resolve(ps, r1);
      A = issue(s0);
    }

    for (int64_t tile = t0;;) {
      step(pr);
      step(ps);
      Rec r3 = load_rec(pr);           // selection record of tile+3
      Slot s2 = resolve(ps, r_next);   // rank rows of tile+2
      B = issue(s_next);               // codes of tile+1
      compute(A);
      if (++tile >= t1) break;
      step(pr);
      step(ps);
      r_next = load_rec(pr);
      s_next = resolve(ps, r3);
      A = issue(s2);
      compute(B);
      if (++tile >= t1) break;
    }

    if (cur_bh >= 0) {
      if (nseg == kGatherSegs) {
        write_stage(1, nseg);
        nseg = 1;
      }
      tile_stage<LPT, MODE>(o, stage[wave][nseg][0], kSource ? stage[wave][nseg][kSets - 1] : nullptr);
      if (lane == 0) seg_bh[wave][nseg] = cur_bh;
      ++nseg;
    }
  }

  // ---- the workgroup's staged segments -> one partial per row and workgroup.  A row's
  // segments are consecutive in wave order (the waves' ranges are consecutive); each row's
  // are combined by the whole workgroup, one thread per partial element:
  //   m = max m_i,  l = sum l_i e^(m_i - m),  acc = sum acc_i e^(m_i - m)
  // (sets whose m is 0 throughout, the selected-PV and aggregate sums, add up unchanged).
  if (lane == 0) seg_n[wave] = nseg;
  __syncthreads();
  {
    const int e = threadIdx.x;
    int q0 = 0, k0 = 0;  // first entry of the next row (entries in wave order, then segment order)
    while (q0 < kWaves && seg_n[q0] > 0) {
      const int bh = seg_bh[q0][k0];
      // entries of this row: (q0, k0), then the first segments of the following waves
      int q1 = q0;
      if (k0 == seg_n[q0] - 1)
        while (q1 + 1 < kWaves && seg_n[q1 + 1] > 0 && seg_bh[q1 + 1][0] == bh) {
          ++q1;
          if (seg_n[q1] > 1) break;  // the row ends inside that wave
        }
      if (e < kPartial) {
        for (int set = 0; set < kSets; ++set) {
          auto part = [&](int q) -> const float* { return stage[q][q == q0 ? k0 : 0][set]; };
          float m = part(q0)[0];
          for (int q = q0 + 1; q <= q1; ++q) m = fmaxf(m, part(q)[0]);
          float r = 0.0f;
          for (int q = q0; q <= q1; ++q) {
            const float* pp = part(q);
            const float sc = pp[0] == -INFINITY ? 0.0f : fast_exp2((pp[0] - m) * kLog2e);
            r = fmaf(sc, pp[e], r);
          }
          a.ws[(static_cast<int64_t>(set) * (a.waves + rows) + gather_slot(blockIdx.x, bh)) * kPartial + e] =
              e == 0 ? m : r;
        }
      }
      // next row: after the last entry used
      if (q1 > q0) {
        q0 = q1;
        k0 = 1;
      } else {
        ++k0;
      }
      if (q0 < kWaves && k0 >= seg_n[q0]) {
        ++q0;
        k0 = 0;
      }
    }
  }
}

// Merge of row bh: slots [f+bh, l+bh] of each partial set (see gather_slot).
__global__ __launch_bounds__(kMergeThreads) void gather_merge_kernel(const float* ws, int waves, int tpr, int nrows,
                                                                     const int32_t* counts, int cap, int tok,
                                                                     float* out, int mode, const float* mass,
                                                                     const float* src, float* src_out) {
  __shared__ MergeLdsBuf S;
  __shared__ int live_red[2][kMergeThreads / kWave];
  const int bh = blockIdx.x, tid = threadIdx.x;
  // the row's live-tile range [rs, re) and the total, as the reader derived them
  int64_t rs = static_cast<int64_t>(bh) * tpr, re = rs + tpr, total = static_cast<int64_t>(nrows) * tpr;
  if (counts != nullptr && nrows <= kLiveRows) {
    int before = 0, all = 0;
    for (int r = tid; r < nrows; r += kMergeThreads) {
      const int n = live_tiles(counts, r, cap, tok);
      all += n;
      if (r < bh) before += n;
    }
    before = wave_sum_int(before);
    all = wave_sum_int(all);
    if ((tid & 63) == 0) {
      live_red[0][tid >> 6] = before;
      live_red[1][tid >> 6] = all;
    }
    __syncthreads();
    before = all = 0;
    for (int w = 0; w < kMergeThreads / kWave; ++w) {
      before += live_red[0][w];
      all += live_red[1][w];
    }
    rs = before;
    re = before + live_tiles(counts, bh, cap, tok);
    total = all;
  }
  const int64_t chunk = (total + waves - 1) / waves * kWaves;  // tiles per reader workgroup
  const int64_t f = rs / chunk, l = (re - 1) / chunk;
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

constexpr int32_t kMaxGatherRows = 1 << 24;  // rows per (b, h) and stream that 32-bit line offsets address

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
  // the readers load row 0 of every stream (and token 0's records) in place of a slot that
  // is absent there, so these must exist even when no prefix is packed yet
  FL_REQUIRE(v.token_capacity > 0 && v.value_meta_token, std::string(who) + ": no token records");
  // a selected row's code line and token record are addressed by 32-bit offsets from the
  // (b, h) row's base: row * 128 and token * 64 bytes
  FL_REQUIRE(v.token_capacity <= kMaxGatherRows, std::string(who) + ": token_capacity above 2^24 tokens per row");
  for (int s = 0; s <= loop; ++s) {
    FL_REQUIRE(v.key_codes[s] && v.key_meta[s] && v.value_codes[s] && v.value_meta[s] && v.key_meta_half[s],
               std::string(who) + ": null stream pointer");
    FL_REQUIRE(v.row_capacity[s] > 0, std::string(who) + ": stream without rows");
    FL_REQUIRE(v.row_capacity[s] <= kMaxGatherRows, std::string(who) + ": row_capacity above 2^24 rows per stream");
    if (s >= 2) FL_REQUIRE(v.rank[s - 2] != nullptr, std::string(who) + ": null rank map");
    FL_REQUIRE(v.value_codes[s] == v.key_codes[s] + kCodeStride / 2,
               std::string(who) + ": value_codes must be the second half of key_codes' lines");
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

constexpr int kLpt = 8;  // lanes per selected slot

// Persistent grid: one wave per tile up to every resident workgroup slot (a small
// selection, e.g. batch one, gets one tile per wave: its waves are latency chains).
int gather_blocks(int rows, int capacity, int occ) {
  const int64_t tiles = static_cast<int64_t>(rows) * (capacity / Lay<kLpt>::kTok);
  const int64_t want = (tiles + kWaves - 1) / kWaves;
  const int64_t slots = static_cast<int64_t>(gather_cu_count()) * std::min(std::max(occ, 1), kGatherMaxResident);
  return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(slots, want)));
}

size_t gather_workspace(int rows, int capacity) {
  const int64_t waves = static_cast<int64_t>(gather_blocks(rows, capacity, kGatherMaxResident)) * kWaves;
  return static_cast<size_t>(2 * (waves + rows)) * kPartial * sizeof(float);
}

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
                     a.waves, a.tpr, rows, a.counts, a.cap, Lay<kLpt>::kTok, a.out, mode, a.mass, a.src, a.src_out);
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
                                         const int32_t* counts, const uint16_t* v_cur, float* out, void* workspace, size_t workspace_bytes,
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
  a.counts = counts;
  a.ws = gather_partials(workspace, rows);
  a.out = out;
  launch_gather<kSelectedPV>(a, rows, static_cast<hipStream_t>(stream));
  FL_LAUNCH_CHECK("fl_decode_selected_pv");
  return FL_OK;
}

extern "C" int32_t fl_decode_attn_sparse_delta(const fl_cache_view* view, int32_t loop, const uint16_t* q,
                                               const uint16_t* k_cur, const uint16_t* v_cur, const int32_t* indices,
                                               const uint8_t* valid, int32_t capacity, const int32_t* counts,
                                               const float* source_output,
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
  a.counts = counts;
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
                                                     int32_t capacity, const int32_t* counts, const float* mass,
                                                     float scaling,
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
  a.counts = counts;
  a.scaling = scaling;
  a.ws = gather_partials(workspace, rows);
  a.out = out;
  a.mass = mass;
  a.src_out = source_output;
  launch_gather<kSparseDeltaFused>(a, rows, static_cast<hipStream_t>(stream));
  FL_LAUNCH_CHECK("fl_decode_attn_sparse_delta_fused");
  return FL_OK;
}
