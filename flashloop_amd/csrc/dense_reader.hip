// J2: fused dense decode reader over the packed int4 residual cache.
//
// logit_t = scaling * q . K_loop[t],  K_loop[t] = sum_{s<=loop} deq(stream s)[t]
// out     = softmax(logits) . V_loop  over [packed prefix ; BF16 tail ; current token]
//
// Layout of the work (one launch + a merge launch):
//   The packed prefixes of all (b,h) form one global sequence of 64-token groups
//   ((b,h)-major).  The grid is persistent: each wave of kPersistBlocks x 4 waves takes
//   one contiguous range of ceil(G / waves) groups and streams it with the next group's
//   loads in flight, flushing a partial (m, l, acc[128]) whenever its range crosses into
//   the next (b,h).  The BF16 tail + current token of each (b,h) is one extra wave task.
//   A merge kernel combines each row's partials (contiguous slots, see partial_slot).
//
// Per-channel K metadata is factored out of the dot product: for group g and stream s,
//   q . deq_s(K)[t] = sum_c (q_c*scale_{g,c}) * code_{t,c} + sum_c q_c*min_{g,c};
// V (per-token metadata) likewise:
//   sum_t p_t*(scale_t*code_t,c + min_t) = sum_t (p_t*scale_t)*code_t,c + sum_t p_t*min_t.
#include "dense_layout.h"
#include "internal.h"

#include <hip/hip_ext.h>

#include <mutex>
#include <vector>

namespace fl {
namespace {
using namespace reader;

struct DenseArgs {
  fl_cache_view v;
  const uint16_t* q;
  const uint16_t* kc;
  const uint16_t* vc;
  float scaling;
  float* logits;
  int64_t logits_stride;
  float* ws;  // partial slots: [waves + B*H] prefix slots, then [B*H] tail slots
  const uint16_t* tail_k;  // tail_key[loop] / tail_value[loop], resolved on the host
  const uint16_t* tail_v;
  int waves;  // persistent waves in the grid
};

// Combine row bh's partials (dense_merge_row).  `pieces` loops were read by one launch
// (dense_pair_kernel: 2): block p*BH + bh merges row bh of piece p.  Defined ahead of the
// reader kernels: with its code placed after them in the code object, the same
// instructions ran 0.8 us longer per launch (cfg3, measured in one process).
__global__ __launch_bounds__(kMergeThreads) void dense_merge_kernel(const float* ws0, const float* ws1, int W,
                                                                    fl_cache_view v, float* out0, float* out1,
                                                                    int pieces) {
  __shared__ DenseMergeLds S;
  dense_merge_row(S, blockIdx.x, ws0, ws1, W, v, out0, out1, pieces);
}

// Position in the work sequence: row (b, h), group gi of gb, row's first unit vs.
struct Cursor {
  int b, h, gi, gb;
  int64_t vs;
};

// Group count of batch b (wave-uniform), kept in a scalar register: from the LDS cache,
// else from the length array (batches past the cache).
__device__ __forceinline__ int row_len(const fl_cache_view& v, const RowLens& rl, int b) {
  b = __builtin_amdgcn_readfirstlane(b);
  if (b < rl.n) return __builtin_amdgcn_readfirstlane(rl.lds[b]);
  return max(min(v.packed_tokens[b], v.token_capacity), 0) / kGroup;
}

// Row containing unit u; gi = u's offset within the row's units.
__device__ __forceinline__ Cursor locate(const fl_cache_view& v, const RowLens& rl, int64_t u) {
  Cursor c{0, 0, 0, 0, 0};
  int64_t base = 0;
  for (int b = 0; b < v.batch; ++b) {
    const int gb = row_len(v, rl, b);
    const int64_t span = kTailUnits + gb;
    const int64_t all = static_cast<int64_t>(v.heads) * span;
    if (u < base + all) {
      c.b = b;
      c.gb = gb;
      c.h = static_cast<int>((u - base) / span);
      c.vs = base + c.h * span;
      c.gi = static_cast<int>(u - c.vs);
      return c;
    }
    base += all;
  }
  c.b = v.batch;
  c.vs = base;
  return c;
}

__device__ __forceinline__ void next_row(Cursor& c, const fl_cache_view& v, const RowLens& rl) {
  c.vs += kTailUnits + c.gb;
  c.gi = 0;
  if (++c.h == v.heads) {
    c.h = 0;
    ++c.b;
  }
  c.gb = c.b < v.batch ? row_len(v, rl, c.b) : 0;
}

// Move to the next prefix group (skipping rows without groups); stops past the end.
__device__ __forceinline__ void advance(Cursor& c, const fl_cache_view& v, const RowLens& rl) {
  ++c.gi;
  while (c.gi >= c.gb && c.b < v.batch) next_row(c, v, rl);
}

__host__ __device__ __forceinline__ int64_t partial_slot(int w, int bh) { return static_cast<int64_t>(w) + bh; }

// ---------------------------------------------------------------------------------
// Prefix groups on the matrix cores.
//
// Both contractions of a 64-token group run as v_mfma_i32_16x16x64_i8 with the nibble
// codes as one operand and a fixed-point image of the float factors as the other:
//   logits: B = K codes [channel x token] (a lane's 16-byte row quarter, split into its
//           even-channel and odd-channel nibbles), A = q*scale per channel;
//   P.V:    B = V codes [token x channel] (read transposed out of LDS with
//           ds_read_b64_tr_b4), A = p*scale per token.
// A float factor x of a group is scaled to X = x*2^24*127/max|x| and rounded to an int32
// (|X| < 2^31); its four bytes, re-centred so every byte is a signed digit, are the four
// A rows m&3 = 0..3 of one MFMA, so the four accumulator rows of a lane hold the digit
// sums of one token (or channel) and sum_k 256^k * D_k rebuilds the dot product with a
// relative error near 2^-25 of the group's largest term -- the fp32 level.
// Per 64 tokens and stream this is 8 + 8 MFMAs instead of ~4.5k VALU operations.
// ---------------------------------------------------------------------------------

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
// 16-byte code chunks as a native vector: copies of HIP's uint4 (a struct) became memcpys
// that SROA left in a per-thread array -- placed in LDS by the compiler, with a store of
// the first loaded chunk that made each wave wait for its first group's loads.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v2i lds_v2i;

constexpr float kFixScale = 127.0f * 16777216.0f;  // 127 * 2^24
constexpr float kLazyRescale = 8.0f;              // rescale when the max grows by > e^8

// Fixed-point digits of X (|X| < 2^31): bytes d0..d3 with X = sum_k d_k*256^k, each d_k
// a signed byte (d0..d2 re-centred by 0x80, d3 the top byte of X + 0x808080).
__device__ __forceinline__ uint32_t fix_digits(float x, float inv) {
  const int32_t X = static_cast<int32_t>(rintf(x * inv));
  return (static_cast<uint32_t>(X) + 0x00808080u) ^ 0x00808080u;
}

__device__ __forceinline__ float undigit(const v4i& d) {
  return fmaf(static_cast<float>(d[3]), 16777216.0f,
              fmaf(static_cast<float>(d[2]), 65536.0f, fmaf(static_cast<float>(d[1]), 256.0f, static_cast<float>(d[0]))));
}

// 4x4 byte transpose inside each quad: lane q returns byte q of the four lanes' words.
__device__ __forceinline__ uint32_t quad_byte_transpose(uint32_t x, int q) {
  const uint32_t p1 = static_cast<uint32_t>(dpp_i<kDppXor1>(static_cast<int>(x)));
  const uint32_t t = __builtin_amdgcn_perm(p1, x, (q & 1) ? 0x03070105u : 0x06020400u);
  const uint32_t p2 = static_cast<uint32_t>(dpp_i<kDppXor2>(static_cast<int>(t)));
  return __builtin_amdgcn_perm(p2, t, (q & 2) ? 0x03020706u : 0x05040100u);
}

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Wave-private LDS of the prefix path.
template <int NS>
struct PrefixLds {
  u32x4 vt[NS][256];          // V codes of the group: entry (i*64 + lane) = row 16i+(lane&15), quarter lane>>4
  uint32_t y[NS][4][2][4][4];  // K-side digits [stream][digit][parity][quarter][4 words of 4 channels]
  uint32_t z[NS][2][4][16];    // V-side digits [stream][half][digit][16 words of 4 tokens]
};

// One 64-token group of one wave: lane = 16*quarter + n.  K/V code loads cover rows
// 16i+n (i = 0..3) at byte quarter `quarter`; V metadata is loaded for the lane's own
// token (row = lane), K metadata for channels 2*lane, 2*lane+1, and q for the same two
// channels (rows change along the global sequence).
template <int NS>
struct GroupSet {
  uint2 km[NS];  // fp16 (scale, min) of channels 2*lane, 2*lane+1
  u32x4 kw[4][NS];
  uint2 vm[NS];  // fp16 (scale, min) of both 64-channel halves of token `lane`
  u32x4 vw[4][NS];
  uint32_t qw;   // bf16 q of channels 2*lane, 2*lane+1
  uint32_t has;  // stream s>=2: bit 5*(s-2)+i row present for tile i, bit 5*(s-2)+4 own token
  int bh, gi;
};

template <int NS>
__device__ __forceinline__ void load_group(GroupSet<NS>& gs, const DenseArgs& a, const Cursor& c) {
  const fl_cache_view& v = a.v;
  const int lane = threadIdx.x & 63, n = lane & 15, quarter = lane >> 4;
  const int bh = c.b * v.heads + c.h, gi = c.gi;
  const int gcap = v.token_capacity / kGroup;
  // Row of token t in stream s (streams 2/3 through the rank map; absent rows read row 0
  // and are masked by `has`), computed where it is used.
  uint32_t has = 0;
  auto row_of = [&](int s, int i) {
    const int t = gi * kGroup + (i < 4 ? 16 * i + n : lane);
    if (s < 2) return t;
    const int r = v.rank[s - 2][static_cast<int64_t>(c.b) * v.token_capacity + t];
    const bool ok = r >= 0 && r < v.row_capacity[s];
    if (ok) has |= 1u << (5 * (s - 2) + i);
    return ok ? r : 0;
  };
  gs.bh = bh;
  gs.gi = gi;
  gs.qw = *reinterpret_cast<const uint32_t*>(a.q + static_cast<int64_t>(bh) * kDim + 2 * lane);
#pragma unroll
  for (int s = 0; s < NS; ++s)
    gs.km[s] = *reinterpret_cast<const uint2*>(v.key_meta_half[s] +
                                               ((static_cast<int64_t>(bh) * gcap + gi) * kDim + 2 * lane) * 2);
  // K and V halves of each 128-byte code line are requested back to back
#pragma unroll
  for (int s = 0; s < NS; ++s)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint8_t* line = v.key_codes[s] + (static_cast<int64_t>(bh) * v.row_capacity[s] + row_of(s, i)) * kCodeStride;
      gs.kw[i][s] = *reinterpret_cast<const u32x4*>(line + 16 * quarter);
      gs.vw[i][s] = *reinterpret_cast<const u32x4*>(v.value_codes[s] - v.key_codes[s] + line + 16 * quarter);
    }
#pragma unroll
  for (int s = 0; s < NS; ++s)
    gs.vm[s] = *reinterpret_cast<const uint2*>(v.value_meta_half[s] +
                                               (static_cast<int64_t>(bh) * v.row_capacity[s] + row_of(s, 4)) * 4);
  gs.has = has;
}

// Wave-level online-softmax state of the prefix path.  m is wave-uniform; l, mu0/mu1
// (sum p*min per V half) are per lane over the lane's tokens; acc[j] holds channel
// 16j + (lane&15) (replicated over the four lane quarters).
struct WaveState {
  float m, l, mu0, mu1;
  float acc[8];
};

__device__ __forceinline__ v4i nib_lo(u32x4 w) {
  return v4i{static_cast<int>(w.x & 0x0F0F0F0Fu), static_cast<int>(w.y & 0x0F0F0F0Fu),
             static_cast<int>(w.z & 0x0F0F0F0Fu), static_cast<int>(w.w & 0x0F0F0F0Fu)};
}
__device__ __forceinline__ v4i nib_hi(u32x4 w) {
  return v4i{static_cast<int>((w.x >> 4) & 0x0F0F0F0Fu), static_cast<int>((w.y >> 4) & 0x0F0F0F0Fu),
             static_cast<int>((w.z >> 4) & 0x0F0F0F0Fu), static_cast<int>((w.w >> 4) & 0x0F0F0F0Fu)};
}

template <int NS, bool LOGITS>
__device__ __forceinline__ void compute_group(const GroupSet<NS>& gs, WaveState& st, PrefixLds<NS>& L,
                                              const DenseArgs& a, float* lgbuf) {
  const int lane = threadIdx.x & 63, n = lane & 15, quarter = lane >> 4, q4 = lane & 3, digit = n & 3;
  wave_lds_sync();  // the previous group's LDS reads are done before these writes
#pragma unroll
  for (int s = 0; s < NS; ++s)
#pragma unroll
    for (int i = 0; i < 4; ++i) L.vt[s][i * 64 + lane] = gs.vw[i][s];

  // ---- K side: y = q*scale per channel (lane: channels 2*lane, 2*lane+1), c_s = q.min
  const float q0 = bf16lo_to_f32(gs.qw) * a.scaling, q1 = bf16hi_to_f32(gs.qw) * a.scaling;
  float y0[NS], y1[NS], c[NS];
  float ymax = 0.0f;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const float ks0 = f16_to_f32(gs.km[s].x & 0xFFFFu), km0 = f16_to_f32(gs.km[s].x >> 16);
    const float ks1 = f16_to_f32(gs.km[s].y & 0xFFFFu), km1 = f16_to_f32(gs.km[s].y >> 16);
    y0[s] = q0 * ks0;
    y1[s] = q1 * ks1;
    ymax = fmaxf(ymax, fmaxf(fabsf(y0[s]), fabsf(y1[s])));
    c[s] = fmaf(q0, km0, q1 * km1);
  }
  // streams 0/1 are present for every token: one reduction of their sum
  // (if constexpr: no index past the one-stream arrays)
  if constexpr (NS > 1) {
    c[0] = wave_sum(c[0] + c[1]);
    c[1] = 0.0f;
  } else {
    c[0] = wave_sum(c[0]);
  }
#pragma unroll
  for (int s = 2; s < NS; ++s) c[s] = wave_sum(c[s]);
  ymax = wave_max(ymax);
  const float yinv = ymax > 0.0f ? kFixScale * __builtin_amdgcn_rcpf(ymax) : 0.0f;
  const float yunit = ymax * (1.0f / kFixScale);
  // channel 2*lane = 32*quarter + 8*(n>>2) + 2*(n&3): parity 0, word (n>>2), byte (n&3)
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    L.y[s][q4][0][quarter][n >> 2] = quad_byte_transpose(fix_digits(y0[s], yinv), q4);
    L.y[s][q4][1][quarter][n >> 2] = quad_byte_transpose(fix_digits(y1[s], yinv), q4);
  }
  wave_lds_sync();
  v4i ae[NS], ao[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    ae[s] = *reinterpret_cast<const v4i*>(&L.y[s][digit][0][quarter][0]);
    ao[s] = *reinterpret_cast<const v4i*>(&L.y[s][digit][1][quarter][0]);
  }
  float lg[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v4i d = {0, 0, 0, 0};
    float cadd = 0.0f;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      u32x4 w = gs.kw[i][s];
      bool ok = true;
      if (s >= 2) {
        ok = (gs.has >> (5 * (s - 2) + i)) & 1u;
        if (!ok) w = u32x4{0u, 0u, 0u, 0u};
      }
      d = __builtin_amdgcn_mfma_i32_16x16x64_i8(ae[s], nib_lo(w), d, 0, 0, 0);
      d = __builtin_amdgcn_mfma_i32_16x16x64_i8(ao[s], nib_hi(w), d, 0, 0, 0);
      if (ok) cadd += c[s];
    }
    lg[i] = fmaf(undigit(d), yunit, cadd);  // token 16i + n
  }

  // ---- softmax of the lane's own token (row = lane: tile `quarter`, position n)
  const float lgo = quarter == 0 ? lg[0] : quarter == 1 ? lg[1] : quarter == 2 ? lg[2] : lg[3];
  if (LOGITS) lgbuf[lane] = lgo;  // staged; written out in batches (stage_flush)
  // the wave's maximum is formed only when some token exceeds m by more than e^8
  if (__ballot(lgo > st.m + kLazyRescale)) {  // wave-uniform
    const float gmax = wave_max(lgo);
    const float alpha = st.m == -INFINITY ? 0.0f : fast_exp2((st.m - gmax) * kLog2e);
    st.l *= alpha;
    st.mu0 *= alpha;
    st.mu1 *= alpha;
#pragma unroll
    for (int j = 0; j < 8; ++j) st.acc[j] *= alpha;
    st.m = gmax;
  }
  const float p = fast_exp2((lgo - st.m) * kLog2e);
  st.l += p;
  float z0[NS], z1[NS];
  float zmax = 0.0f;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const bool ok = s < 2 || ((gs.has >> (5 * (s - 2) + 4)) & 1u);
    const float vs0 = f16_to_f32(gs.vm[s].x & 0xFFFFu), vm0 = f16_to_f32(gs.vm[s].x >> 16);
    const float vs1 = f16_to_f32(gs.vm[s].y & 0xFFFFu), vm1 = f16_to_f32(gs.vm[s].y >> 16);
    z0[s] = ok ? p * vs0 : 0.0f;
    z1[s] = ok ? p * vs1 : 0.0f;
    if (ok) {
      st.mu0 = fmaf(p, vm0, st.mu0);
      st.mu1 = fmaf(p, vm1, st.mu1);
    }
    zmax = fmaxf(zmax, fmaxf(z0[s], z1[s]));
  }
  zmax = wave_max(zmax);
  const float zinv = zmax > 0.0f ? kFixScale * __builtin_amdgcn_rcpf(zmax) : 0.0f;
  const float zunit = zmax * (1.0f / kFixScale);
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    L.z[s][0][q4][lane >> 2] = quad_byte_transpose(fix_digits(z0[s], zinv), q4);
    L.z[s][1][q4][lane >> 2] = quad_byte_transpose(fix_digits(z1[s], zinv), q4);
  }
  wave_lds_sync();

  // ---- P.V: channel tile j (16j .. 16j+15); lane (quarter, n) supplies row 16*quarter +
  // sigma(n) so that the unpacked nibbles come out in token order 16*quarter + 0..15.
  const int sig = (n & 8) | ((n & 1) << 2) | ((n >> 1) & 3);
  v4i az[NS][2];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    az[s][0] = *reinterpret_cast<const v4i*>(&L.z[s][0][digit][4 * quarter]);
    az[s][1] = *reinterpret_cast<const v4i*>(&L.z[s][1][digit][4 * quarter]);
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    v4i d = {0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const char* base = reinterpret_cast<const char*>(&L.vt[s][0]) +
                         (quarter * 64 + 16 * (j >> 1) + sig) * 16 + 8 * (j & 1);
      const v2i t = __builtin_amdgcn_ds_read_tr4_b64_v2i32(
          (lds_v2i*)((__attribute__((address_space(3))) char*)(base)));
      const uint4 w = make_uint4(static_cast<uint32_t>(t[0]), static_cast<uint32_t>(t[0]) >> 4,
                                 static_cast<uint32_t>(t[1]), static_cast<uint32_t>(t[1]) >> 4);
      const v4i bop = {static_cast<int>(w.x & 0x0F0F0F0Fu), static_cast<int>(w.y & 0x0F0F0F0Fu),
                       static_cast<int>(w.z & 0x0F0F0F0Fu), static_cast<int>(w.w & 0x0F0F0F0Fu)};
      d = __builtin_amdgcn_mfma_i32_16x16x64_i8(az[s][j >> 2], bop, d, 0, 0, 0);
    }
    st.acc[j] = fmaf(undigit(d), zunit, st.acc[j]);
  }
}

__device__ __forceinline__ void reset_state(WaveState& st) {
  st.m = -INFINITY;
  st.l = st.mu0 = st.mu1 = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) st.acc[j] = 0.0f;
}

// BF16 tail of the loop + the current token (virtual row tl) of row bh, by one wave:
// lane = 4*row + quarter, 16 tokens per pass, 32 channels per lane; the 16 quad states
// are merged through the wave's LDS (`comb`).
template <bool LOGITS>
__device__ void wave_tail(const DenseArgs& a, int bh, float (*comb)[kDim]) {
  const fl_cache_view& v = a.v;
  const int lane = threadIdx.x & 63, quarter = lane & 3, row = lane >> 2;
  const int b = bh / v.heads;
  const int Tp = row_groups(v, b) * kGroup;
  const int tl = min(max(v.tail_tokens[b], 0), v.tail_capacity);
  const uint16_t* tk = a.tail_k + static_cast<int64_t>(bh) * v.tail_capacity * kDim;
  const uint16_t* tv = a.tail_v + static_cast<int64_t>(bh) * v.tail_capacity * kDim;
  const uint16_t* ck = a.kc + static_cast<int64_t>(bh) * kDim;
  const uint16_t* cv = a.vc + static_cast<int64_t>(bh) * kDim;
  float* lrow = LOGITS ? a.logits + static_cast<int64_t>(bh) * a.logits_stride : nullptr;
  float qr[32];
#pragma unroll
  for (int c = 0; c < 32; ++c) qr[c] = bf16_to_f32(a.q[static_cast<int64_t>(bh) * kDim + 32 * quarter + c]) * a.scaling;
  QuadState st;
  st.m = -INFINITY;
  st.l = 0.0f;
  st.mu = 0.0f;
#pragma unroll
  for (int c = 0; c < 32; ++c) st.acc[c] = 0.0f;
  const int n = tl + 1;
  // 16 tokens per step (lane = 4*row + quarter).  The next step's rows are requested
  // while a step computes, from two named register sets (a copy of a set still in flight
  // would wait for it); every load is unconditional: rows past the end read the current
  // token's row and are masked.
  struct Rows {
    u32x4 k[4], v[4];
  };
  auto fetch = [&](Rows& r, int base) __attribute__((always_inline)) {
    const int vt = base + row;
    const uint16_t* kr = (vt < tl) ? tk + static_cast<int64_t>(vt) * kDim : ck;
    const uint16_t* vr = (vt < tl) ? tv + static_cast<int64_t>(vt) * kDim : cv;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      r.k[k] = *reinterpret_cast<const u32x4*>(kr + 32 * quarter + 8 * k);
      r.v[k] = *reinterpret_cast<const u32x4*>(vr + 32 * quarter + 8 * k);
    }
  };
  auto step = [&](const Rows& r, int base) __attribute__((always_inline)) {
    const int vt = base + row;
    const bool valid = vt < n;
    float d = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const u32x4 w = r.k[k];
      d = fmaf(qr[8 * k + 0], bf16lo_to_f32(w.x), d);
      d = fmaf(qr[8 * k + 1], bf16hi_to_f32(w.x), d);
      d = fmaf(qr[8 * k + 2], bf16lo_to_f32(w.y), d);
      d = fmaf(qr[8 * k + 3], bf16hi_to_f32(w.y), d);
      d = fmaf(qr[8 * k + 4], bf16lo_to_f32(w.z), d);
      d = fmaf(qr[8 * k + 5], bf16hi_to_f32(w.z), d);
      d = fmaf(qr[8 * k + 6], bf16lo_to_f32(w.w), d);
      d = fmaf(qr[8 * k + 7], bf16hi_to_f32(w.w), d);
    }
    d = quad_sum(d);
    float lg = valid ? d : -INFINITY;
    if (LOGITS && quarter == 0 && valid && Tp + vt < a.logits_stride) lrow[Tp + vt] = lg;
    float p;
    online_update(st, &lg, &p, 1);
    p = valid ? p : 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t ws[4] = {r.v[k].x, r.v[k].y, r.v[k].z, r.v[k].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        st.acc[8 * k + 2 * e] = fmaf(p, bf16lo_to_f32(ws[e]), st.acc[8 * k + 2 * e]);
        st.acc[8 * k + 2 * e + 1] = fmaf(p, bf16hi_to_f32(ws[e]), st.acc[8 * k + 2 * e + 1]);
      }
    }
  };
  // Peeled like the prefix loop: the steady-state body has no exit between a set's fetch
  // and its use, so the compiler's waits count only the younger set's loads (an exit
  // between them made it wait for every load, one full round trip per 16 rows).
  const int steps = (n + 15) / 16;
  Rows ra, rb;
  fetch(ra, 0);
  int s = 0;
  for (; s + 2 < steps; s += 2) {
    fetch(rb, 16 * s + 16);
    step(ra, 16 * s);
    fetch(ra, 16 * s + 32);
    step(rb, 16 * s + 16);
  }
  if (steps - s == 2) {
    fetch(rb, 16 * s + 16);
    step(ra, 16 * s);
    step(rb, 16 * s + 16);
  } else {
    step(ra, 16 * s);
  }
  const float M = wave_max(st.m);  // finite: the current token is always present
  const float f = st.m == -INFINITY ? 0.0f : fast_exp2((st.m - M) * kLog2e);
  wave_lds_sync();  // earlier LDS use of this wave is complete
#pragma unroll
  for (int c = 0; c < 32; ++c) comb[row][32 * quarter + c] = st.acc[c] * f;
  const float L = wave_sum(quarter == 0 ? st.l * f : 0.0f);
  wave_lds_sync();
  float* part = a.ws + (static_cast<int64_t>(a.waves) + v.batch * v.heads + bh) * kPartial;  // tail slot
  float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    s0 += comb[r][2 * lane];
    s1 += comb[r][2 * lane + 1];
  }
  part[2 + 2 * lane] = s0;
  part[3 + 2 * lane] = s1;
  if (lane == 0) {
    part[0] = M;
    part[1] = L;
  }
}

template <int NS>
union WaveLds {
  PrefixLds<NS> p;
  float comb[16][kDim];
};

// Outputs of the prefix stream (logits of every group, one partial per row segment) are
// staged in wave-private LDS and written after the wave's last load.  On gfx9-family
// GPUs stores and loads share the in-order vmcnt counter, so a store issued mid-stream
// holds up every later load wait until its write is acknowledged -- under a saturated
// read stream that costs far more than the store's bytes.
constexpr int kStageGroups = 64;  // logits of 64 groups (16 KB) per wave
constexpr int kStageSegs = 4;     // partials of up to 4 row segments per wave

// Row segments of the staged outputs live in wave-private LDS (a register array indexed
// by a runtime count would be placed in scratch memory, whose accesses are vector memory
// operations too).
struct SegMeta {
  int bh, gi0, first, count;
};

// Write the staged logits and partials of segments [0, n); the partial of segment n-1 is
// skipped when it is still open.
template <bool LOGITS>
__device__ __forceinline__ void stage_flush(const DenseArgs& a, const SegMeta* seg, int n, const float* lgbuf,
                                            const float (*pbuf)[kPartial], int w, bool last_open) {
  const int lane = threadIdx.x & 63;
  wave_lds_sync();
  for (int k = 0; k < n; ++k) {
    const SegMeta m = seg[k];
    if (LOGITS) {
      float* dst = a.logits + static_cast<int64_t>(m.bh) * a.logits_stride + static_cast<int64_t>(m.gi0) * kGroup;
      const float* src = lgbuf + m.first * kGroup;
      // a row never writes past its stride (device lengths above the host maxima)
      const int64_t room = a.logits_stride - static_cast<int64_t>(m.gi0) * kGroup;
      const int cnt = static_cast<int>(min(static_cast<int64_t>(m.count * kGroup), max(room, int64_t{0})));
      // 16 bytes per lane and store (a row's logits start on a 256-byte boundary of the
      // group grid; the stride may leave a row 4-byte aligned only: then dword stores)
      const int c4 = (reinterpret_cast<uintptr_t>(dst) & 15u) == 0 ? cnt >> 2 : 0;
      for (int e = lane; e < c4; e += kWave)
        reinterpret_cast<float4*>(dst)[e] = reinterpret_cast<const float4*>(src)[e];
      for (int e = 4 * c4 + lane; e < cnt; e += kWave) dst[e] = src[e];
    }
    if (!(last_open && k == n - 1)) {
      float* part = a.ws + partial_slot(w, m.bh) * kPartial;
      for (int e = lane; e < kPartial; e += kWave) part[e] = pbuf[k][e];
    }
  }
  wave_lds_sync();
}

// Stage the wave state of the current segment into pbuf[slot].
__device__ __forceinline__ void stage_partial(const WaveState& st, float* part) {
  const int lane = threadIdx.x & 63, n = lane & 15;
  const float L = wave_sum(st.l), mu0 = wave_sum(st.mu0), mu1 = wave_sum(st.mu1);
  if (lane < 16) {
#pragma unroll
    for (int j = 0; j < 8; ++j) part[2 + 16 * j + n] = st.acc[j] + (j < 4 ? mu0 : mu1);
  }
  if (lane == 0) {
    part[0] = st.m;
    part[1] = L;
  }
}

// LDS of one reader wave: every array a wave touches lives in its own block, at fixed
// offsets, so no wave's staging overlaps another's whatever loop body each is running.
template <int NS, bool LOGITS>
struct WaveBlock {
  WaveLds<NS> sh;
  float lg[LOGITS ? kStageGroups * kGroup : 1];
  float ps[kStageSegs][kPartial];
  SegMeta seg[kStageSegs];
};

// The LDS of one reader workgroup.
template <int NS, bool LOGITS>
struct ReaderLds {
  WaveBlock<NS, LOGITS> w[kWaves];
};

// Wave-private block of the pair launch: loop 1 and loop 2 bodies view the same bytes
// through their own types; a wave runs the bodies one after the other.
union PairWaveBlock {
  WaveBlock<1, false> l1;
  WaveBlock<2, true> l2;
};

// Wave w's units [u0, u1) of one loop's work sequence; W is the calling wave's LDS block.
template <int NS, bool LOGITS>
__device__ __forceinline__ void dense_range(const DenseArgs& a, WaveBlock<NS, LOGITS>& W, const RowLens& rl, int w,
                                            int64_t u0, int64_t u1) {
  if (u0 >= u1) return;
  const fl_cache_view& v = a.v;

  // Tails whose first unit lies in [u0, u1), then the count of prefix groups in range.
  Cursor c = locate(v, rl, u0);
  int my = 0;
  {
    Cursor t = c;
    bool first = true;
    while (t.b < v.batch && t.vs < u1) {
      if (t.vs >= u0) wave_tail<LOGITS>(a, t.b * v.heads + t.h, W.sh.comb);
      const int64_t p0 = max(t.vs + kTailUnits, first ? u0 : t.vs), p1 = min(t.vs + kTailUnits + t.gb, u1);
      if (p1 > p0) my += static_cast<int>(p1 - p0);
      first = false;
      next_row(t, v, rl);
    }
  }
  if (my == 0) return;
  // first prefix group in range
  Cursor ld = c;
  ld.gi = max(c.gi - kTailUnits, 0);
  while (ld.gi >= ld.gb && ld.b < v.batch) next_row(ld, v, rl);

  WaveState st;
  reset_state(st);
  // Current segment in registers (wave-uniform); closed segments in LDS.
  int nseg = 0, used = 0, cur_bh = -1, cur_gi0 = 0, cur_first = 0, cur_count = 0;
  float* lgbuf = W.lg;
  float(*pbuf)[kPartial] = W.ps;
  SegMeta* seg = W.seg;
  auto close_seg = [&]() {
    stage_partial(st, pbuf[nseg - 1]);
    if ((threadIdx.x & 63) == 0) seg[nseg - 1] = SegMeta{cur_bh, cur_gi0, cur_first, cur_count};
  };
  auto run = [&](const GroupSet<NS>& gs) __attribute__((always_inline)) {
    if (gs.bh != cur_bh) {
      if (nseg > 0) close_seg();
      if (nseg == kStageSegs || (LOGITS && used == kStageGroups)) {  // rare: stage full
        stage_flush<LOGITS>(a, seg, nseg, lgbuf, pbuf, w, false);
        nseg = 0;
        used = 0;
      }
      reset_state(st);
      cur_bh = gs.bh;
      cur_gi0 = gs.gi;
      cur_first = used;
      cur_count = 0;
      ++nseg;
    } else if (LOGITS && used == kStageGroups) {  // rare: logits stage full mid-segment
      if ((threadIdx.x & 63) == 0) seg[nseg - 1] = SegMeta{cur_bh, cur_gi0, cur_first, cur_count};
      stage_flush<LOGITS>(a, seg, nseg, lgbuf, pbuf, w, true);
      nseg = 1;
      used = 0;
      cur_gi0 = gs.gi;
      cur_first = 0;
      cur_count = 0;
    }
    compute_group<NS, LOGITS>(gs, st, W.sh.p, a, lgbuf + (LOGITS ? used * kGroup : 0));
    ++used;
    ++cur_count;
  };
  // Ping-pong: the next group's loads are in flight while a group computes.  The
  // steady-state body issues its loads unconditionally: a load under a branch makes the
  // waitcnt merge at the join wait for every outstanding load (vmcnt(0)).
  GroupSet<NS> set0, set1;
  load_group<NS>(set0, a, ld);
  advance(ld, v, rl);
  int k = 0;
  for (; k + 2 < my; k += 2) {
    load_group<NS>(set1, a, ld);
    advance(ld, v, rl);
    run(set0);
    load_group<NS>(set0, a, ld);
    advance(ld, v, rl);
    run(set1);
  }
  if (my - k == 2) {
    load_group<NS>(set1, a, ld);
    run(set0);
    run(set1);
  } else {
    run(set0);
  }
  close_seg();
  stage_flush<LOGITS>(a, seg, nseg, lgbuf, pbuf, w, false);
}

// At most two waves per SIMD: a tighter register budget makes the compiler spill the
// ping-pong load sets to scratch (measured: the loop-1 reader 126 -> 154 us).
template <int NS, bool LOGITS>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 2))) void dense_reader_kernel(DenseArgs a) {
  __shared__ ReaderLds<NS, LOGITS> L;
  __shared__ int lens[kLenCache];
  const fl_cache_view& v = a.v;
  // wave-uniform: the work cursor and every length lookup stay in scalar registers
  const int w = blockIdx.x * kWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  for (int i = threadIdx.x; i < min(v.batch, kLenCache); i += kThreads) lens[i] = row_groups(v, i);
  __syncthreads();
  const RowLens rl{lens, min(v.batch, kLenCache)};
  const int64_t U = total_units(v, rl);
  const int64_t chunk = chunk_of(U, a.waves);
  const int64_t u0 = static_cast<int64_t>(w) * chunk;
  dense_range<NS, LOGITS>(a, L.w[threadIdx.x >> 6], rl, w, u0, min(u0 + chunk, U));
}

// Loops 1 and 2 of a decode step in one persistent launch (loop 2 with logits).  Their
// work sequences are equal (streams 0 and 1 both cover the packed prefix); laid end to
// end, they are split evenly over the waves, so the spread of the waves' end times is
// paid once instead of once per loop.  Units [0, U) are loop 1's, [U, 2U) loop 2's; a
// wave's partials go to its loop's workspace at the slots of its global wave index.
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 2))) void dense_pair_kernel(DenseArgs a0,
                                                                                                    DenseArgs a1) {
  __shared__ PairWaveBlock L[kWaves];
  __shared__ int lens[kLenCache];
  const fl_cache_view& v = a0.v;
  const int w = blockIdx.x * kWaves + (threadIdx.x >> 6);
  PairWaveBlock& mine = L[threadIdx.x >> 6];
  for (int i = threadIdx.x; i < min(v.batch, kLenCache); i += kThreads) lens[i] = row_groups(v, i);
  __syncthreads();
  const RowLens rl{lens, min(v.batch, kLenCache)};
  const int64_t U = total_units(v, rl);
  const int64_t chunk = chunk_of(2 * U, a0.waves);
  const int64_t u0 = static_cast<int64_t>(w) * chunk, u1 = min(u0 + chunk, 2 * U);
  dense_range<1, false>(a0, mine.l1, rl, w, u0, min(u1, U));
  // The two bodies view the wave's block through different types, which type-based
  // alias analysis takes as disjoint: without a compiler barrier, loop 2's first LDS
  // writes could be scheduled above loop 1's last staging reads.  The memory clobber
  // orders every access; the wait completes this wave's loop-1 LDS reads.  Other waves
  // never touch this block.
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  dense_range<2, true>(a1, mine.l2, rl, w, max(u0, U) - U, max(u1, U) - U);
}


int cu_count() {
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

// Resident workgroups per CU of a reader instantiation (cached per device).
template <int NS, bool LOGITS>
int occupancy() {
  static std::mutex mu;
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 1;
  std::lock_guard<std::mutex> g(mu);
  if (cached[dev] == 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, dense_reader_kernel<NS, LOGITS>, kThreads, 0) != hipSuccess ||
        n <= 0)
      n = 1;
    cached[dev] = n;
  }
  return cached[dev];
}

int occupancy_pair() {
  static std::mutex mu;
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 1;
  std::lock_guard<std::mutex> g(mu);
  if (cached[dev] == 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, dense_pair_kernel, kThreads, 0) != hipSuccess || n <= 0) n = 1;
    cached[dev] = n;
  }
  return cached[dev];
}

int occupancy_of(int loop, bool logits) {
  switch (loop * 2 + (logits ? 1 : 0)) {
    case 0: return occupancy<1, false>();
    case 1: return occupancy<1, true>();
    case 2: return occupancy<2, false>();
    case 3: return occupancy<2, true>();
    case 4: return occupancy<3, false>();
    case 5: return occupancy<3, true>();
    case 6: return occupancy<4, false>();
    default: return occupancy<4, true>();
  }
}

constexpr int kMaxResident = 2;  // workgroups per CU any reader instantiation can hold
constexpr int kProfilePair = 4;  // fl_profile_dense_reader code of the pair launch

// ---- measurement hook (fl_profile_dense_reader): a HIP event pair on the reader kernel's
// own dispatch (hipExtLaunchKernel: the events take the kernel's start and end times, with
// no marker packet before or after it on the stream)
struct ReaderProfile {
  int loop = -1, want = 0, used = 0;
  bool armed = false;  // the current call records (set by profile_before)
  std::vector<hipEvent_t> start, stop;
};
struct EventPair {
  hipEvent_t start = nullptr, stop = nullptr;
};
std::mutex g_prof_mu;
ReaderProfile g_prof;

void profile_free() {
  for (hipEvent_t e : g_prof.start) (void)hipEventDestroy(e);
  for (hipEvent_t e : g_prof.stop) (void)hipEventDestroy(e);
  g_prof = ReaderProfile{};
}

// The event pair this launch records into (none: not profiling, or under capture).
EventPair profile_before(hipStream_t st, int loop) {
  std::lock_guard<std::mutex> g(g_prof_mu);
  g_prof.armed = false;
  if (g_prof.used >= g_prof.want || (g_prof.loop >= 0 && g_prof.loop != loop)) return {};
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return {};
  g_prof.armed = true;
  return EventPair{g_prof.start[g_prof.used], g_prof.stop[g_prof.used]};
}

void profile_after(bool launched) {
  std::lock_guard<std::mutex> g(g_prof_mu);
  if (!g_prof.armed) return;
  g_prof.armed = false;
  if (launched) ++g_prof.used;
}

// Launch of one reader kernel, on its own events when profiling.
template <typename K, typename... Args>
void launch_reader(K kernel, dim3 grid, dim3 block, hipStream_t st, const EventPair& ev, Args... args) {
  if (ev.start)
    hipExtLaunchKernelGGL(kernel, grid, block, 0, st, ev.start, ev.stop, 0, args...);
  else
    hipLaunchKernelGGL(kernel, grid, block, 0, st, args...);
}

// Persistent grid: every resident 4-wave workgroup slot of the GPU, fewer when the
// cache is small.  Sized from the capacity, not the current lengths, so that the launch
// (and a graph that captured it) stays valid while the prefixes grow.
int persist_blocks(const fl_cache_view& v, int occ) {
  const int64_t rows = static_cast<int64_t>(v.batch) * v.heads;
  const int64_t gmax = rows * (v.token_capacity / kGroup);
  const int64_t want = (gmax + rows * kTailUnits + kWaves - 1) / kWaves;
  const int64_t slots = static_cast<int64_t>(cu_count()) * std::min(std::max(occ, 1), kMaxResident);
  return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(slots, want)));
}

}  // namespace
}  // namespace fl

extern "C" int32_t fl_profile_dense_reader(int32_t loop, int32_t launches) {
  using namespace fl;
  clear_error();
  FL_REQUIRE(launches >= 0 && launches <= 100000, "fl_profile_dense_reader: launches out of range");
  std::lock_guard<std::mutex> g(g_prof_mu);
  profile_free();
  if (launches == 0) return FL_OK;
  g_prof.loop = loop;
  g_prof.want = launches;
  g_prof.start.resize(launches);
  g_prof.stop.resize(launches);
  for (int i = 0; i < launches; ++i) {
    if (hipEventCreate(&g_prof.start[i]) != hipSuccess || hipEventCreate(&g_prof.stop[i]) != hipSuccess) {
      g_prof.start.resize(i);
      g_prof.stop.resize(i);
      profile_free();
      set_error("fl_profile_dense_reader: hipEventCreate failed");
      return FL_E_LAUNCH;
    }
  }
  return FL_OK;
}

extern "C" int32_t fl_profile_dense_reader_read(float* total_ms, int32_t* launches) {
  using namespace fl;
  clear_error();
  FL_REQUIRE(total_ms && launches, "fl_profile_dense_reader_read: null output");
  std::lock_guard<std::mutex> g(g_prof_mu);
  float sum = 0.0f;
  for (int i = 0; i < g_prof.used; ++i) {
    float ms = 0.0f;
    if (hipEventSynchronize(g_prof.stop[i]) != hipSuccess ||
        hipEventElapsedTime(&ms, g_prof.start[i], g_prof.stop[i]) != hipSuccess) {
      set_error("fl_profile_dense_reader_read: event query failed");
      return FL_E_LAUNCH;
    }
    sum += ms;
  }
  *total_ms = sum;
  *launches = g_prof.used;
  g_prof.used = 0;
  return FL_OK;
}

extern "C" size_t fl_decode_attn_dense_workspace(const fl_cache_view* view) {
  using namespace fl;
  if (!view) return 0;
  const int64_t rows = static_cast<int64_t>(view->batch) * view->heads;
  const int64_t waves = static_cast<int64_t>(persist_blocks(*view, kMaxResident)) * kWaves;
  return static_cast<size_t>(waves + 2 * rows) * kPartial * sizeof(float);
}

namespace fl {
namespace {
// Argument checks of one dense read (loop `loop`, logits optional).
int32_t dense_checks(const fl_cache_view* view, int32_t loop, const uint16_t* q, const uint16_t* k_cur,
                     const uint16_t* v_cur, float* out, float* logits, int64_t logits_stride, void* workspace) {
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
    FL_REQUIRE(v.key_codes[s] && v.key_meta_half[s] && v.value_codes[s] && v.value_meta_half[s],
               "fl_decode_attn_dense: null stream pointer");
    // an absent row of streams 2/3 reads row 0 (masked)
    FL_REQUIRE(v.row_capacity[s] > 0, "fl_decode_attn_dense: stream without rows");
    if (s >= 2) FL_REQUIRE(v.rank[s - 2] != nullptr, "fl_decode_attn_dense: null rank map");
  }
  FL_REQUIRE(logits == nullptr || logits_stride >= static_cast<int64_t>(v.max_packed_tokens) + v.max_tail_tokens + 1,
             "fl_decode_attn_dense: logits_stride smaller than the key count");
  FL_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 16 == 0, "fl_decode_attn_dense: workspace must be 16-byte aligned");
  return FL_OK;
}
}  // namespace
}  // namespace fl

namespace fl {
namespace {
// One dense read on a checked workspace: the reader launch and (with `merge`) its merge;
// *waves receives the reader's grid size in waves.
int32_t dense_launch(const fl_cache_view& v, int32_t loop, const uint16_t* q, const uint16_t* k_cur,
                     const uint16_t* v_cur, float scaling, float* out, float* logits, int64_t logits_stride,
                     float* ws, hipStream_t st, bool merge = true, int* waves = nullptr) {
  DenseArgs a{};
  a.v = v;
  a.q = q;
  a.kc = k_cur;
  a.vc = v_cur;
  a.scaling = scaling;
  a.logits = logits;
  a.logits_stride = logits_stride;
  a.ws = ws;
  a.tail_k = v.tail_key[loop];
  a.tail_v = v.tail_value[loop];
  const int blocks = persist_blocks(v, occupancy_of(loop, logits != nullptr));
  a.waves = blocks * kWaves;
  // a row has at most waves + 1 prefix partials (see partial_slot) plus its tail partial
  FL_REQUIRE(a.waves + 2 <= kMergeMaxParts, "fl_decode_attn_dense: too many persistent waves for one merge");
  const dim3 grid(blocks), block(kThreads);
  const EventPair ev = profile_before(st, loop);
  const bool lg = logits != nullptr;
  switch (loop * 2 + (lg ? 1 : 0)) {
    case 0: launch_reader(dense_reader_kernel<1, false>, grid, block, st, ev, a); break;
    case 1: launch_reader(dense_reader_kernel<1, true>, grid, block, st, ev, a); break;
    case 2: launch_reader(dense_reader_kernel<2, false>, grid, block, st, ev, a); break;
    case 3: launch_reader(dense_reader_kernel<2, true>, grid, block, st, ev, a); break;
    case 4: launch_reader(dense_reader_kernel<3, false>, grid, block, st, ev, a); break;
    case 5: launch_reader(dense_reader_kernel<3, true>, grid, block, st, ev, a); break;
    case 6: launch_reader(dense_reader_kernel<4, false>, grid, block, st, ev, a); break;
    default: launch_reader(dense_reader_kernel<4, true>, grid, block, st, ev, a); break;
  }
  profile_after(hipPeekAtLastError() == hipSuccess);
  FL_LAUNCH_CHECK("fl_decode_attn_dense(reader)");
  if (waves) *waves = a.waves;
  if (!merge) return FL_OK;
  hipLaunchKernelGGL(dense_merge_kernel, dim3(v.batch * v.heads), dim3(kMergeThreads), 0, st,
                     static_cast<const float*>(a.ws), static_cast<const float*>(a.ws), a.waves, v, out, out, 1);
  FL_LAUNCH_CHECK("fl_decode_attn_dense(merge)");
  return FL_OK;
}

// ---- the allocation-free entry point's scratch: partials of fl_decode_attn_dense_noalloc.
// One copy per GPU, held until the process ends.  Host code never uses the array's name
// as an address (on the host it is a stand-in symbol): each device's address comes from
// hipGetSymbolAddress, called once per device with that device current.
constexpr size_t kScratchBytes = size_t(8) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {nullptr};

int32_t scratch_ptr(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("fl_decode_attn_dense_noalloc: no current HIP device");
    return FL_E_LAUNCH;
  }
  std::lock_guard<std::mutex> g(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      set_error(std::string("fl_decode_attn_dense_noalloc: hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
      return FL_E_LAUNCH;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return FL_OK;
}
}  // namespace
}  // namespace fl

extern "C" int32_t fl_decode_attn_dense(const fl_cache_view* view, int32_t loop, const uint16_t* q,
                                        const uint16_t* k_cur, const uint16_t* v_cur, float scaling, float* out,
                                        float* logits, int64_t logits_stride, void* workspace,
                                        size_t workspace_bytes, void* stream) {
  using namespace fl;
  clear_error();
  if (const int32_t rc = dense_checks(view, loop, q, k_cur, v_cur, out, logits, logits_stride, workspace); rc != FL_OK)
    return rc;
  FL_REQUIRE(workspace_bytes >= fl_decode_attn_dense_workspace(view), "fl_decode_attn_dense: workspace too small");
  return dense_launch(*view, loop, q, k_cur, v_cur, scaling, out, logits, logits_stride, static_cast<float*>(workspace),
                      static_cast<hipStream_t>(stream));
}

extern "C" int32_t fl_decode_attn_dense_select(const fl_cache_view* view, int32_t loop, const uint16_t* q,
                                               const uint16_t* k_cur, const uint16_t* v_cur, float scaling,
                                               float* out, float* logits, int64_t logits_stride, double fraction,
                                               int32_t capacity, int32_t* indices, uint8_t* valid, float* mass,
                                               float* weights, int32_t* counts, int32_t* nonfinite, void* workspace,
                                               size_t workspace_bytes, void* stream) {
  using namespace fl;
  clear_error();
  if (const int32_t rc = dense_checks(view, loop, q, k_cur, v_cur, out, logits, logits_stride, workspace); rc != FL_OK)
    return rc;
  FL_REQUIRE(logits != nullptr, "fl_decode_attn_dense_select: logits are required");
  FL_REQUIRE(indices && valid && mass && weights, "fl_decode_attn_dense_select: null selection output");
  FL_REQUIRE(capacity > 0, "fl_decode_attn_dense_select: bad capacity");
  FL_REQUIRE(fraction > 0.0 && fraction <= 1.0, "fl_decode_attn_dense_select: fraction must be in (0, 1]");
  FL_REQUIRE(select_merge_fits(logits_stride, fraction), "fl_decode_attn_dense_select: logits_stride above 35840 "
             "keys or a selection above 8192 keys (use fl_decode_attn_dense + fl_decode_topk)");
  FL_REQUIRE(workspace_bytes >= fl_decode_attn_dense_workspace(view), "fl_decode_attn_dense_select: workspace too small");
  hipStream_t st = static_cast<hipStream_t>(stream);
  float* ws = static_cast<float*>(workspace);
  int waves = 0;
  if (const int32_t rc = dense_launch(*view, loop, q, k_cur, v_cur, scaling, out, logits, logits_stride, ws, st,
                                      false, &waves);
      rc != FL_OK)
    return rc;
  return launch_select_merge(*view, ws, waves, out, logits, logits_stride, fraction, capacity, indices, valid, mass,
                             weights, counts, nonfinite, st);
}

extern "C" size_t fl_decode_attn_dense_noalloc_max_bytes(void) { return fl::kScratchBytes; }

extern "C" int32_t fl_decode_attn_dense_noalloc(const fl_cache_view* view, int32_t loop, const uint16_t* q,
                                                const uint16_t* k_cur, const uint16_t* v_cur, float scaling,
                                                float* out, float* logits, int64_t logits_stride, void* stream) {
  using namespace fl;
  clear_error();
  FL_REQUIRE(view != nullptr, "fl_decode_attn_dense_noalloc: view is null");
  const size_t need = fl_decode_attn_dense_workspace(view);
  if (need > kScratchBytes) {
    set_error("fl_decode_attn_dense_noalloc: the cache needs " + std::to_string(need) +
              " bytes of partials, more than the static scratch holds (" + std::to_string(kScratchBytes) +
              " bytes, about 7000 (batch, head) rows); use fl_decode_attn_dense with a workspace");
    return FL_E_CAPACITY;
  }
  void* ws = nullptr;
  if (const int32_t rc = scratch_ptr(&ws); rc != FL_OK) return rc;
  if (const int32_t rc = dense_checks(view, loop, q, k_cur, v_cur, out, logits, logits_stride, ws); rc != FL_OK)
    return rc;
  return dense_launch(*view, loop, q, k_cur, v_cur, scaling, out, logits, logits_stride, static_cast<float*>(ws),
                      static_cast<hipStream_t>(stream));
}

namespace {
// Byte offset of the second loop's partials in a pair workspace (256-byte aligned).
size_t pair_half(const fl_cache_view* view) { return (fl_decode_attn_dense_workspace(view) + 255) / 256 * 256; }
}  // namespace

extern "C" size_t fl_decode_attn_dense_pair_workspace(const fl_cache_view* view) {
  return view ? 2 * pair_half(view) : 0;
}

extern "C" int32_t fl_decode_attn_dense_pair(const fl_cache_view* view, const uint16_t* q0, const uint16_t* k_cur0,
                                             const uint16_t* v_cur0, float* out0, const uint16_t* q1,
                                             const uint16_t* k_cur1, const uint16_t* v_cur1, float* out1,
                                             float scaling, float* logits1, int64_t logits_stride, void* workspace,
                                             size_t workspace_bytes, void* stream) {
  using namespace fl;
  clear_error();
  if (const int32_t rc = dense_checks(view, 0, q0, k_cur0, v_cur0, out0, nullptr, 0, workspace); rc != FL_OK) return rc;
  if (const int32_t rc = dense_checks(view, 1, q1, k_cur1, v_cur1, out1, logits1, logits_stride, workspace); rc != FL_OK)
    return rc;
  FL_REQUIRE(logits1 != nullptr, "fl_decode_attn_dense_pair: loop-2 logits are required");
  FL_REQUIRE(workspace_bytes >= fl_decode_attn_dense_pair_workspace(view), "fl_decode_attn_dense_pair: workspace too small");
  const fl_cache_view& v = *view;
  DenseArgs a[2]{};
  const uint16_t* qs[2] = {q0, q1};
  const uint16_t* ks[2] = {k_cur0, k_cur1};
  const uint16_t* vs[2] = {v_cur0, v_cur1};
  const int blocks = persist_blocks(v, occupancy_pair());
  for (int r = 0; r < 2; ++r) {
    a[r].v = v;
    a[r].q = qs[r];
    a[r].kc = ks[r];
    a[r].vc = vs[r];
    a[r].scaling = scaling;
    a[r].logits = r == 1 ? logits1 : nullptr;
    a[r].logits_stride = r == 1 ? logits_stride : 0;
    a[r].ws = reinterpret_cast<float*>(static_cast<char*>(workspace) + r * pair_half(view));
    a[r].tail_k = v.tail_key[r];
    a[r].tail_v = v.tail_value[r];
    a[r].waves = blocks * kWaves;
  }
  FL_REQUIRE(a[0].waves + 2 <= kMergeMaxParts, "fl_decode_attn_dense_pair: too many persistent waves for one merge");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const EventPair ev = profile_before(st, kProfilePair);
  launch_reader(dense_pair_kernel, dim3(blocks), dim3(kThreads), st, ev, a[0], a[1]);
  profile_after(hipPeekAtLastError() == hipSuccess);
  FL_LAUNCH_CHECK("fl_decode_attn_dense_pair(reader)");
  hipLaunchKernelGGL(dense_merge_kernel, dim3(2 * v.batch * v.heads), dim3(kMergeThreads), 0, st,
                     static_cast<const float*>(a[0].ws), static_cast<const float*>(a[1].ws), a[0].waves, v, out0, out1, 2);
  FL_LAUNCH_CHECK("fl_decode_attn_dense_pair(merge)");
  return FL_OK;
}
