// Decode-step model kernels: the per-layer work around the cache readers, fused so that
// one decode step of a layer and loop is eight launches instead of ~60 (the step of
// flashloop/engine.py:396-537 on an Ouro-shaped sandwich-norm layer).
//
//  * fl_gemv_bf16 -- y[m, n] = sum_k x[m, k] * W[n, k] for m < M <= 8 (nn.Linear weights,
//    bf16, row-major [N, K]); fp32 accumulation; epilogues: plain bf16 out, f32 out of the
//    bf16-rounded value (lm_head(...).float()), + bf16 addend, SwiGLU of a gate and an up
//    matrix, or rotary embedding of q/k (and a plain v) from three matrices at once.
//  * fl_norm_chain -- the residual/RMSNorm chain between two GEMVs of one row:
//    h = r + n_a(x); optionally h = n_f(h); z = n_b(h).
//
// Every rounding to bf16 happens where the torch modules round (Linear output, RMSNorm
// output, each binary op of rotate-half RoPE, SiLU, the SwiGLU product, residual adds).
//
// GEMV work split: a workgroup of kGemvWaves waves owns kRows output rows and splits K
// between its waves (each wave streams 64 contiguous 16-byte chunks of each row per
// step); the waves reduce their partial dots in registers (DPP) and combine through LDS.
// The grid has N / kRows workgroups (>= 512 for every matrix of the model), so every CU
// has several row blocks of weights in flight.  Memory-bound: bytes = N * K * 2 + M * K.
#include "fl_common.h"

namespace fl {
namespace {

constexpr int kGemvWaves = 4;
constexpr int kGemvThreads = kGemvWaves * kWave;
constexpr int kRows = 4;  // output rows per workgroup
constexpr int kMaxM = 8;

enum GemvEpi : int { kEpiPlain = 0, kEpiF32 = 1, kEpiAdd = 2, kEpiSwiGlu = 3, kEpiRope = 4 };

struct GemvArgs {
  const void* x;  // [M, K] bf16, or f32 (rounded to bf16 on load) when x_f32
  int64_t x_stride;
  int x_f32;
  int M, K, N;  // N: rows of each matrix
  const uint16_t* w[3];  // plain/add/f32: w[0]; swiglu: gate w[0], up w[1]; rope: q, k, v
  void* y[3];            // outputs [M, N] (row stride y_stride); rope: q, k, v
  int64_t y_stride;
  const uint16_t* addend;  // kEpiAdd: [M, N] bf16 (row stride addend_stride)
  int64_t addend_stride;
  const uint16_t* cos;  // kEpiRope: [M, 128] bf16 tables of each row's position
  const uint16_t* sin;
  int head_dim;
};

__device__ __forceinline__ float bf16_round(float v) { return round_bf16(v); }

__device__ __forceinline__ void unpack8(const uint4& u, float* f) {
  f[0] = bf16lo_to_f32(u.x);
  f[1] = bf16hi_to_f32(u.x);
  f[2] = bf16lo_to_f32(u.y);
  f[3] = bf16hi_to_f32(u.y);
  f[4] = bf16lo_to_f32(u.z);
  f[5] = bf16hi_to_f32(u.z);
  f[6] = bf16lo_to_f32(u.w);
  f[7] = bf16hi_to_f32(u.w);
}

// A raw buffer resource over `bytes` bytes at p (wave-uniform): loads past the end (or
// from a resource of size 0) return zero.  Word 3 is the gfx9 raw-buffer format.
using BufRes = __amdgpu_buffer_rsrc_t;
__device__ __forceinline__ BufRes buf_res(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, static_cast<int>(bytes), 0x00020000);
}
__device__ __forceinline__ uint4 buf_load16(BufRes r, uint32_t off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(off), 0, 0));
}

// x chunk q (8 values) of row m, as the bf16 values the Linear sees
template <bool XF32>
__device__ __forceinline__ void load_x8(const GemvArgs& a, int m, int q, float* f) {
  if (XF32) {
    const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(a.x) + m * a.x_stride + 8 * q);
    const float4 u = p[0], v = p[1];
    f[0] = bf16_round(u.x);
    f[1] = bf16_round(u.y);
    f[2] = bf16_round(u.z);
    f[3] = bf16_round(u.w);
    f[4] = bf16_round(v.x);
    f[5] = bf16_round(v.y);
    f[6] = bf16_round(v.z);
    f[7] = bf16_round(v.w);
  } else {
    unpack8(*reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.x) + m * a.x_stride + 8 * q), f);
  }
}

// Rows of workgroup g.  Plain: 4 consecutive rows of w[0].  SwiGLU: 2 consecutive rows,
// each of the gate and of the up matrix.  RoPE: matrix g / (N/4); within it the rotary
// pair rows {c, c+1, c+64, c+65} of one head, c even < 64.
template <int EPI>
__device__ __forceinline__ void block_rows(const GemvArgs& a, int g, const uint16_t** rp, int* mat, int* n0) {
  if (EPI == kEpiSwiGlu) {
    const int n = 2 * g;
    rp[0] = a.w[0] + static_cast<int64_t>(n) * a.K;
    rp[1] = a.w[0] + static_cast<int64_t>(n + 1) * a.K;
    rp[2] = a.w[1] + static_cast<int64_t>(n) * a.K;
    rp[3] = a.w[1] + static_cast<int64_t>(n + 1) * a.K;
    *mat = 0;
    *n0 = n;
  } else if (EPI == kEpiRope) {
    const int per = a.N / kRows;
    const int m = g / per, gi = g - m * per;
    const int half = a.head_dim / 2, pairs = half / 2;  // row groups per head
    const int head = gi / pairs, c = 2 * (gi - head * pairs);
    const int n = head * a.head_dim + c;
    const uint16_t* w = a.w[m];
    rp[0] = w + static_cast<int64_t>(n) * a.K;
    rp[1] = w + static_cast<int64_t>(n + 1) * a.K;
    rp[2] = w + static_cast<int64_t>(n + half) * a.K;
    rp[3] = w + static_cast<int64_t>(n + half + 1) * a.K;
    *mat = m;
    *n0 = n;
  } else {
    const int n = kRows * g;
#pragma unroll
    for (int r = 0; r < kRows; ++r) rp[r] = a.w[0] + static_cast<int64_t>(n + r) * a.K;
    *mat = 0;
    *n0 = n;
  }
}

// Cross-wave reduction of the partial dots and the epilogue (wave 0, lane m writes row m).
template <int MT, int EPI>
__device__ __forceinline__ void gemv_finish(const GemvArgs& a, float (*acc)[kRows], float (*red)[MT][kRows], int mat,
                                            int n0) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
      const float s = wave_sum(acc[m][r]);
      if (lane == 0) red[wave][m][r] = s;
    }
  __syncthreads();
  if (wave != 0 || lane >= a.M) return;
  const int m = lane;
  float v[kRows];
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < kGemvWaves; ++w) s += red[w][m < MT ? m : 0][r];
    v[r] = bf16_round(s);  // the Linear's bf16 output
  }
  const int64_t yo = static_cast<int64_t>(m) * a.y_stride + n0;
  if (EPI == kEpiF32) {
    float* y = static_cast<float*>(a.y[0]) + yo;
#pragma unroll
    for (int r = 0; r < kRows; ++r) y[r] = v[r];
  } else if (EPI == kEpiPlain || EPI == kEpiAdd) {
    uint16_t* y = static_cast<uint16_t*>(a.y[0]) + yo;
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
      float o = v[r];
      if (EPI == kEpiAdd) o = o + bf16_to_f32(a.addend[static_cast<int64_t>(m) * a.addend_stride + n0 + r]);
      y[r] = f32_to_bf16_rne(o);
    }
  } else if (EPI == kEpiSwiGlu) {
    // silu(gate) rounds to bf16 (F.silu on bf16), then the product rounds
    uint16_t* y = static_cast<uint16_t*>(a.y[0]) + yo;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const float g = v[r], u = v[2 + r];
      const float s = bf16_round(g / (1.0f + expf(-g)));
      y[r] = f32_to_bf16_rne(s * u);
    }
  } else {  // rope: rows (c, c+1) and (c+64, c+65); rotate_half(x)[c] = -x[c+64], [c+64] = x[c]
    uint16_t* y = static_cast<uint16_t*>(a.y[mat]) + yo;
    const int half = a.head_dim / 2;
    if (mat == 2) {
      y[0] = f32_to_bf16_rne(v[0]);
      y[1] = f32_to_bf16_rne(v[1]);
      y[half] = f32_to_bf16_rne(v[2]);
      y[half + 1] = f32_to_bf16_rne(v[3]);
    } else {
      const int c = (n0 % a.head_dim);
      const uint16_t* cs = a.cos + static_cast<int64_t>(m) * a.head_dim;
      const uint16_t* sn = a.sin + static_cast<int64_t>(m) * a.head_dim;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const float lo = v[e], hi = v[2 + e];
        const float cl = bf16_to_f32(cs[c + e]), sl = bf16_to_f32(sn[c + e]);
        const float ch = bf16_to_f32(cs[c + half + e]), sh = bf16_to_f32(sn[c + half + e]);
        y[e] = f32_to_bf16_rne(bf16_round(lo * cl) + bf16_round(-hi * sl));
        y[half + e] = f32_to_bf16_rne(bf16_round(hi * ch) + bf16_round(lo * sh));
      }
    }
  }
}

template <int MT, int EPI, bool XF32>
__global__ __launch_bounds__(kGemvThreads) void gemv_kernel(GemvArgs a) {
  __shared__ float red[kGemvWaves][MT][kRows];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint16_t* rp[kRows];
  int mat, n0;
  block_rows<EPI>(a, blockIdx.x, rp, &mat, &n0);
  float acc[MT][kRows];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int r = 0; r < kRows; ++r) acc[m][r] = 0.0f;
  const int nq = a.K / 8;  // 16-byte chunks per row
  // chunk q = j*256 + wave*64 + lane: each wave reads 1 KB contiguous per row and step
  constexpr int kStep = kGemvWaves * kWave;
  int q = wave * kWave + lane;
  // two steps per iteration keep 8 row loads in flight per lane
  for (; q + kStep < nq; q += 2 * kStep) {
    uint4 w0[kRows], w1[kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
      w0[r] = reinterpret_cast<const uint4*>(rp[r])[q];
      w1[r] = reinterpret_cast<const uint4*>(rp[r])[q + kStep];
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      if (m < a.M) {
        float x0[8], x1[8];
        load_x8<XF32>(a, m, q, x0);
        load_x8<XF32>(a, m, q + kStep, x1);
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
          float f[8];
          unpack8(w0[r], f);
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[m][r] = fmaf(x0[e], f[e], acc[m][r]);
          unpack8(w1[r], f);
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[m][r] = fmaf(x1[e], f[e], acc[m][r]);
        }
      }
    }
  }
  if (q < nq) {
    uint4 w0[kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r) w0[r] = reinterpret_cast<const uint4*>(rp[r])[q];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      if (m < a.M) {
        float x0[8];
        load_x8<XF32>(a, m, q, x0);
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
          float f[8];
          unpack8(w0[r], f);
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[m][r] = fmaf(x0[e], f[e], acc[m][r]);
        }
      }
    }
  }
  gemv_finish<MT, EPI>(a, acc, red, mat, n0);
}

// The GEMV with every chunk a thread owns (S of them per row, K <= S * 2048) requested
// at once as bounds-checked buffer loads: chunks past K and rows past M read as zero, so
// no load sits under a branch (the compiler's wait after a branch join drains every
// outstanding load).  Same accumulation order as gemv_kernel.
template <int MT, int EPI, bool XF32, int S>
__global__ __launch_bounds__(kGemvThreads) void gemv_flat_kernel(GemvArgs a) {
  __shared__ float red[kGemvWaves][MT][kRows];
  const uint16_t* rp[kRows];
  int mat, n0;
  block_rows<EPI>(a, blockIdx.x, rp, &mat, &n0);
  constexpr int kStep = kGemvThreads;
  constexpr uint32_t kXb = XF32 ? 4u : 2u;  // bytes per x element
  const uint32_t q = threadIdx.x;
  uint4 wv[S][kRows];
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    const BufRes wr = buf_res(rp[r], static_cast<uint32_t>(a.K) * 2u);
#pragma unroll
    for (int s = 0; s < S; ++s) wv[s][r] = buf_load16(wr, 16u * (q + s * kStep));
  }
  uint4 xv[MT][S][XF32 ? 2 : 1];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    const bool live = m < a.M;
    const BufRes xr = buf_res(live ? static_cast<const char*>(a.x) + static_cast<int64_t>(m) * a.x_stride * kXb : nullptr,
                              live ? static_cast<uint32_t>(a.K) * kXb : 0u);
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const uint32_t off = 8u * kXb * (q + s * kStep);
      xv[m][s][0] = buf_load16(xr, off);
      if (XF32) xv[m][s][XF32 ? 1 : 0] = buf_load16(xr, off + 16u);
    }
  }
  float acc[MT][kRows];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int r = 0; r < kRows; ++r) acc[m][r] = 0.0f;
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int s = 0; s < S; ++s) {
      float x[8];
      if (XF32) {
        const uint4 u = xv[m][s][0], v = xv[m][s][XF32 ? 1 : 0];
        const uint32_t w8[8] = {u.x, u.y, u.z, u.w, v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = bf16_round(__uint_as_float(w8[e]));
      } else {
        unpack8(xv[m][s][0], x);
      }
#pragma unroll
      for (int r = 0; r < kRows; ++r) {
        float f[8];
        unpack8(wv[s][r], f);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[m][r] = fmaf(x[e], f[e], acc[m][r]);
      }
    }
  gemv_finish<MT, EPI>(a, acc, red, mat, n0);
}

// ---------------------------------------------------------------------------------
// Residual / RMSNorm chain of one row (one workgroup per row).  Thread t owns the
// 8-value chunks t, t + 256, ... of the row; every global load (x, r and the three
// weight rows) is issued before the first reduction, so the chain costs one memory
// round trip plus its block reductions.
// RMSNorm(x) = bf16(w * (x * rsqrt(mean(x^2) + eps))) in fp32, as the model's module.
constexpr int kNormThreads = 256;
constexpr int kNormChunks = 4;  // 8-value chunks per thread: D <= 8192

struct NormArgs {
  int D;
  float eps;
  const uint16_t* x;   // [M, D] or null (then h = r)
  const uint16_t* r;   // [M, D] residual / input
  const uint16_t* wa;  // norm of x
  const uint16_t* wf;  // optional norm of h (replaces h)
  const uint16_t* wb;  // optional norm of h -> z
  uint16_t* h_out;     // optional
  uint16_t* z_out;     // optional
  int64_t stride;      // row stride of every [M, D] tensor
};

constexpr int kNormWaves = kNormThreads / kWave;

// Block sums through two LDS buffers used in turn: reduction k writes buffer k & 1 and
// every wave reads it before it reaches the barrier of reduction k + 1, so buffer k & 1 is
// free again for reduction k + 2 -- one barrier per sum.
struct BlockSum {
  float (*red)[kNormWaves];
  int phase;
  __device__ __forceinline__ float operator()(float v) {
    float* r = red[phase & 1];
    ++phase;
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) r[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < kNormWaves; ++i) s += r[i];
    return s;
  }
};

// v <- RMSNorm(v) with weight chunks w (8 values per chunk), rounded to bf16
template <int NC>
__device__ __forceinline__ void rms_apply(float (*v)[8], const uint4* w, int nc, int D, float eps, BlockSum& bs) {
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < NC; ++i)
    if (i < nc)
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(v[i][e], v[i][e], ss);
  const float inv = rsqrtf(bs(ss) / static_cast<float>(D) + eps);
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    float wf[8];
    unpack8(w[i], wf);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[i][e] = bf16_round(wf[e] * (v[i][e] * inv));
  }
}

__device__ __forceinline__ uint4 pack8(const float* f) {
  uint4 u;
  u.x = static_cast<uint32_t>(f32_to_bf16_rne(f[0])) | (static_cast<uint32_t>(f32_to_bf16_rne(f[1])) << 16);
  u.y = static_cast<uint32_t>(f32_to_bf16_rne(f[2])) | (static_cast<uint32_t>(f32_to_bf16_rne(f[3])) << 16);
  u.z = static_cast<uint32_t>(f32_to_bf16_rne(f[4])) | (static_cast<uint32_t>(f32_to_bf16_rne(f[5])) << 16);
  u.w = static_cast<uint32_t>(f32_to_bf16_rne(f[6])) | (static_cast<uint32_t>(f32_to_bf16_rne(f[7])) << 16);
  return u;
}

// The chain of row `base` (element offset): h = r (+ n_a(x)), optionally h = n_f(h),
// written to h_out when write_h; then z = n_b(h) when n_b is given.  chain_load issues the
// loads of this thread's chunks t, t + 256, ...; chain_finish leaves z (or h without n_b)
// in v as bf16 values.  All kNormThreads threads must call chain_finish (block reductions).
template <int NC>
struct ChainIn {
  uint4 xr[NC], rr[NC], wa[NC], wf[NC], wb[NC];
};

template <int NC>
__device__ __forceinline__ void chain_load(const NormArgs& a, int64_t base, ChainIn<NC>& in) {
  const int nq = a.D / 8;
  const int nc = (nq - static_cast<int>(threadIdx.x) + kNormThreads - 1) / kNormThreads;  // my chunks
  // Buffer loads sized to each operand (size 0 when absent): chunks past the row read as
  // zero without a branch.  A load under a branch would make the compiler's wait at the
  // join drain every outstanding load, including a caller's loads issued after these.
  (void)nc;
  const uint32_t row = static_cast<uint32_t>(a.D) * 2u;
  const BufRes r = buf_res(a.r + base, row);
  const BufRes x = buf_res(a.x ? a.x + base : nullptr, a.x ? row : 0u);
  const BufRes wa = buf_res(a.x ? a.wa : nullptr, a.x ? row : 0u);
  const BufRes wf = buf_res(a.wf, a.wf ? row : 0u);
  const BufRes wb = buf_res(a.wb, a.wb ? row : 0u);
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const uint32_t off = 16u * static_cast<uint32_t>(threadIdx.x + i * kNormThreads);
    in.rr[i] = buf_load16(r, off);
    in.xr[i] = buf_load16(x, off);
    in.wa[i] = buf_load16(wa, off);
    in.wf[i] = buf_load16(wf, off);
    in.wb[i] = buf_load16(wb, off);
  }
}

template <int NC>
__device__ __forceinline__ void chain_finish(const NormArgs& a, int64_t base, bool write_h, const ChainIn<NC>& in,
                                             float (*h)[8], BlockSum& bs) {
  const int nc = (a.D / 8 - static_cast<int>(threadIdx.x) + kNormThreads - 1) / kNormThreads;
#pragma unroll
  for (int i = 0; i < NC; ++i) unpack8(in.rr[i], h[i]);
  if (a.x != nullptr) {
    float xv[NC][8];
#pragma unroll
    for (int i = 0; i < NC; ++i) unpack8(in.xr[i], xv[i]);
    rms_apply<NC>(xv, in.wa, nc, a.D, a.eps, bs);
#pragma unroll
    for (int i = 0; i < NC; ++i)
#pragma unroll
      for (int e = 0; e < 8; ++e) h[i][e] = bf16_round(h[i][e] + xv[i][e]);
  }
  if (a.wf != nullptr) rms_apply<NC>(h, in.wf, nc, a.D, a.eps, bs);
  if (write_h && a.h_out != nullptr) {
#pragma unroll
    for (int i = 0; i < NC; ++i)
      if (i < nc) reinterpret_cast<uint4*>(a.h_out + base)[threadIdx.x + i * kNormThreads] = pack8(h[i]);
  }
  if (a.wb != nullptr) rms_apply<NC>(h, in.wb, nc, a.D, a.eps, bs);
}

template <int NC>
__device__ __forceinline__ void chain_row(const NormArgs& a, int64_t base, bool write_h, float (*h)[8], BlockSum& bs) {
  ChainIn<NC> in;
  chain_load<NC>(a, base, in);
  chain_finish<NC>(a, base, write_h, in, h, bs);
}

template <int NC>
__global__ __launch_bounds__(kNormThreads) void norm_chain_kernel(NormArgs a) {
  __shared__ float red[2][kNormWaves];
  BlockSum bs{red, 0};
  const int64_t base = static_cast<int64_t>(blockIdx.x) * a.stride;
  const int nc = (a.D / 8 - static_cast<int>(threadIdx.x) + kNormThreads - 1) / kNormThreads;
  float h[NC][8];
  chain_row<NC>(a, base, true, h, bs);
  if (a.wb != nullptr) {
#pragma unroll
    for (int i = 0; i < NC; ++i)
      if (i < nc) reinterpret_cast<uint4*>(a.z_out + base)[threadIdx.x + i * kNormThreads] = pack8(h[i]);
  }
}

// GEMV whose input rows are the chain's output, computed in the prologue of every
// workgroup (bit-identical to norm_chain_kernel: same chunk ownership, same reductions);
// workgroup 0 writes h.  The weight chunks are requested before the chain so its loads
// and reductions run under their latency.  K <= kChainMaxK (each thread's x chunks are the
// chunks it normalises, so z stays in registers).
constexpr int kChainSteps = 2;
constexpr int kChainMaxK = kChainSteps * kGemvThreads * 8;
static_assert(kGemvThreads == kNormThreads, "the chain prologue maps one GEMV thread to one chain thread");

template <int MT, int EPI, int NC>
__global__ __launch_bounds__(kGemvThreads) void gemv_chain_kernel(GemvArgs a, NormArgs c) {
  __shared__ float red[kGemvWaves][MT][kRows];
  __shared__ float nred[2][kNormWaves];
  BlockSum bs{nred, 0};
  const uint16_t* rp[kRows];
  int mat, n0;
  block_rows<EPI>(a, blockIdx.x, rp, &mat, &n0);
  const int nq = a.K / 8;
  constexpr int kStep = kGemvThreads;
  const int q = threadIdx.x;
  // row 0's chain inputs are requested before the weights: the wave's loads return in
  // order, so the chain (two block reductions) then runs while the weights are in flight
  ChainIn<NC> in0;
  chain_load<NC>(c, 0, in0);
  __builtin_amdgcn_sched_barrier(0);  // keep the issue order: chain inputs, then weights
  uint4 wv[NC][kRows];  // weight chunks past K (buffer bounds) read as zero, no branch
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    const BufRes wr = buf_res(rp[r], static_cast<uint32_t>(a.K) * 2u);
#pragma unroll
    for (int s = 0; s < NC; ++s) wv[s][r] = buf_load16(wr, 16u * static_cast<uint32_t>(q + s * kStep));
  }
  float acc[MT][kRows];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int r = 0; r < kRows; ++r) acc[m][r] = 0.0f;
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    if (m < a.M) {
      float z[NC][8];
      if (m == 0)
        chain_finish<NC>(c, 0, blockIdx.x == 0, in0, z, bs);
      else
        chain_row<NC>(c, static_cast<int64_t>(m) * c.stride, blockIdx.x == 0, z, bs);
#pragma unroll
      for (int s = 0; s < NC; ++s)
        if (q + s * kStep < nq)
#pragma unroll
          for (int r = 0; r < kRows; ++r) {
            float f[8];
            unpack8(wv[s][r], f);
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[m][r] = fmaf(z[s][e], f[e], acc[m][r]);
          }
    }
  }
  gemv_finish<MT, EPI>(a, acc, red, mat, n0);
}

// ---------------------------------------------------------------------------------
// Decode append: the step's K/V rows of the four loops go to each sequence's tail at its
// device length, the loop-3/4 activity flags of that row are set, and the length is
// incremented -- one workgroup per sequence, so the increment follows its own copies.
constexpr int kAppendThreads = 256;

struct AppendArgs {
  fl_cache_view v;
  const uint16_t* k[4];  // [B*H, 128] bf16 rows of the step, per loop
  const uint16_t* val[4];
  uint8_t* active[2];  // [B, tail_capacity] loop-3/4 tail activity
  int32_t* tail_tokens;  // the view's tail lengths, written
};

__global__ __launch_bounds__(kAppendThreads) void append_tail_kernel(AppendArgs a) {
  const fl_cache_view& v = a.v;
  const int b = blockIdx.x;
  constexpr int kChunks = kDim / 8;   // 16-byte chunks per row
  const int per = v.heads * kChunks;  // chunks of one tensor for this sequence
  // tensor t: loop t & 3, K for t < 4; t is a compile-time index in every use below (a
  // runtime index into the argument arrays would load each pointer from memory first)
  auto src_of = [&](int t, int i) __attribute__((always_inline)) {
    const uint16_t* base = t < 4 ? a.k[t & 3] : a.val[t & 3];
    const int h = i / kChunks, c = i - h * kChunks;
    return reinterpret_cast<const uint4*>(base + (static_cast<int64_t>(b) * v.heads + h) * kDim) + c;
  };
  auto dst_of = [&](int t, int i, int pos) __attribute__((always_inline)) {
    uint16_t* base = static_cast<uint16_t*>(t < 4 ? v.tail_key[t & 3] : v.tail_value[t & 3]);
    const int h = i / kChunks, c = i - h * kChunks;
    return reinterpret_cast<uint4*>(base + ((static_cast<int64_t>(b) * v.heads + h) * v.tail_capacity + pos) * kDim) +
           c;
  };
  // chunk threadIdx.x of each of the 8 tensors is requested before the first store (the
  // rows do not depend on the tail length, loaded alongside): one memory round trip
  const int pos = v.tail_tokens[b];
  const int i0 = threadIdx.x;
  uint4 held[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) held[t] = i0 < per ? *src_of(t, i0) : make_uint4(0, 0, 0, 0);
  if (pos < 0 || pos >= v.tail_capacity) return;  // the host rolls over before the tail is full
#pragma unroll
  for (int t = 0; t < 8; ++t)
    if (i0 < per) *dst_of(t, i0, pos) = held[t];
  for (int i = i0 + kAppendThreads; i < per; i += kAppendThreads)  // more than 16 heads
#pragma unroll
    for (int t = 0; t < 8; ++t) *dst_of(t, i, pos) = *src_of(t, i);
  if (threadIdx.x < 2) a.active[threadIdx.x][static_cast<int64_t>(b) * v.tail_capacity + pos] = 1;
  __syncthreads();
  if (threadIdx.x == 0) a.tail_tokens[b] = pos + 1;
}

template <int MT, int EPI, bool XF32>
void launch_gemv_x(const GemvArgs& a, int blocks, hipStream_t st) {
  const int steps = (a.K + kGemvThreads * 8 - 1) / (kGemvThreads * 8);
  const dim3 g(blocks), t(kGemvThreads);
  switch (steps) {
    case 1: hipLaunchKernelGGL((gemv_flat_kernel<MT, EPI, XF32, 1>), g, t, 0, st, a); break;
    case 2: hipLaunchKernelGGL((gemv_flat_kernel<MT, EPI, XF32, 2>), g, t, 0, st, a); break;
    case 3: hipLaunchKernelGGL((gemv_flat_kernel<MT, EPI, XF32, 3>), g, t, 0, st, a); break;
    case 4: hipLaunchKernelGGL((gemv_flat_kernel<MT, EPI, XF32, 4>), g, t, 0, st, a); break;
    default: hipLaunchKernelGGL((gemv_kernel<MT, EPI, XF32>), g, t, 0, st, a); break;  // K > 8192
  }
}

template <int MT, int EPI>
void launch_gemv_m(const GemvArgs& a, int blocks, hipStream_t st) {
  if (MT > 2) {  // the flat form would hold MT x S x-chunks in registers
    if (a.x_f32)
      hipLaunchKernelGGL((gemv_kernel<MT, EPI, true>), dim3(blocks), dim3(kGemvThreads), 0, st, a);
    else
      hipLaunchKernelGGL((gemv_kernel<MT, EPI, false>), dim3(blocks), dim3(kGemvThreads), 0, st, a);
  } else if (a.x_f32) {
    launch_gemv_x<(MT > 2 ? 2 : MT), EPI, true>(a, blocks, st);
  } else {
    launch_gemv_x<(MT > 2 ? 2 : MT), EPI, false>(a, blocks, st);
  }
}

template <int EPI>
void launch_gemv(const GemvArgs& a, int blocks, hipStream_t st) {
  if (a.M <= 1)
    launch_gemv_m<1, EPI>(a, blocks, st);
  else if (a.M <= 2)
    launch_gemv_m<2, EPI>(a, blocks, st);
  else if (a.M <= 4)
    launch_gemv_m<4, EPI>(a, blocks, st);
  else
    launch_gemv_m<8, EPI>(a, blocks, st);
}

template <int EPI, int NC>
void launch_gemv_chain_nc(const GemvArgs& a, const NormArgs& c, int blocks, hipStream_t st) {
  if (a.M <= 1)
    hipLaunchKernelGGL((gemv_chain_kernel<1, EPI, NC>), dim3(blocks), dim3(kGemvThreads), 0, st, a, c);
  else if (a.M <= 2)
    hipLaunchKernelGGL((gemv_chain_kernel<2, EPI, NC>), dim3(blocks), dim3(kGemvThreads), 0, st, a, c);
  else if (a.M <= 4)
    hipLaunchKernelGGL((gemv_chain_kernel<4, EPI, NC>), dim3(blocks), dim3(kGemvThreads), 0, st, a, c);
  else
    hipLaunchKernelGGL((gemv_chain_kernel<8, EPI, NC>), dim3(blocks), dim3(kGemvThreads), 0, st, a, c);
}

template <int EPI>
void launch_gemv_chain(const GemvArgs& a, const NormArgs& c, int blocks, hipStream_t st) {
  if (a.K <= kGemvThreads * 8)
    launch_gemv_chain_nc<EPI, 1>(a, c, blocks, st);
  else
    launch_gemv_chain_nc<EPI, kChainSteps>(a, c, blocks, st);
}

// Argument checks and GemvArgs shared by both GEMV entry points.
int32_t make_gemv_args(GemvArgs& a, const void* x, int32_t x_is_f32, int64_t x_stride, int32_t m, int32_t k,
                       const uint16_t* const* weights, int32_t n, int32_t epilogue, void* const* outputs,
                       int64_t out_stride, const uint16_t* addend, int64_t addend_stride, const uint16_t* rope_cos,
                       const uint16_t* rope_sin, int32_t head_dim, const char* who) {
  const std::string w(who);
  FL_REQUIRE(x && weights && outputs, w + ": null x/weights/outputs");
  FL_REQUIRE(m >= 1 && m <= kMaxM, w + ": rows of x must be 1..8");
  FL_REQUIRE(k > 0 && k % 8 == 0 && n > 0 && n % kRows == 0, w + ": K must be a multiple of 8, N of 4");
  FL_REQUIRE(x_stride >= k && out_stride >= n, w + ": bad row strides");
  FL_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0 && (x_stride * (x_is_f32 ? 4 : 2)) % 16 == 0,
             w + ": x rows must be 16-byte aligned");
  FL_REQUIRE(epilogue >= kEpiPlain && epilogue <= kEpiRope, w + ": unknown epilogue");
  const int nmat = epilogue == kEpiRope ? 3 : (epilogue == kEpiSwiGlu ? 2 : 1);
  for (int i = 0; i < nmat; ++i) {
    FL_REQUIRE(weights[i] != nullptr && reinterpret_cast<uintptr_t>(weights[i]) % 16 == 0,
               w + ": weights must be non-null and 16-byte aligned");
    a.w[i] = weights[i];
  }
  const int nout = epilogue == kEpiRope ? 3 : 1;
  for (int i = 0; i < nout; ++i) {
    FL_REQUIRE(outputs[i] != nullptr, w + ": null output");
    a.y[i] = outputs[i];
  }
  if (epilogue == kEpiAdd) FL_REQUIRE(addend != nullptr && addend_stride >= n, w + ": bad addend");
  if (epilogue == kEpiSwiGlu) FL_REQUIRE(n % 2 == 0, w + ": SwiGLU needs an even N");
  if (epilogue == kEpiRope)
    FL_REQUIRE(rope_cos && rope_sin && head_dim >= 8 && head_dim % 8 == 0 && n % head_dim == 0,
               w + ": rope needs cos/sin tables and N a multiple of head_dim (multiple of 8)");
  a.x = x;
  a.x_f32 = x_is_f32 ? 1 : 0;
  a.x_stride = x_stride;
  a.M = m;
  a.K = k;
  a.N = n;
  a.y_stride = out_stride;
  a.addend = addend;
  a.addend_stride = addend_stride;
  a.cos = rope_cos;
  a.sin = rope_sin;
  a.head_dim = head_dim;
  return FL_OK;
}

int gemv_blocks(int epilogue, int n) {
  return epilogue == kEpiSwiGlu ? n / 2 : (epilogue == kEpiRope ? 3 * (n / kRows) : n / kRows);
}

}  // namespace
}  // namespace fl

extern "C" int32_t fl_gemv_bf16(const void* x, int32_t x_is_f32, int64_t x_stride, int32_t m, int32_t k,
                                const uint16_t* const* weights, int32_t n, int32_t epilogue, void* const* outputs,
                                int64_t out_stride, const uint16_t* addend, int64_t addend_stride,
                                const uint16_t* rope_cos, const uint16_t* rope_sin, int32_t head_dim, void* stream) {
  using namespace fl;
  clear_error();
  GemvArgs a{};
  const int32_t rc = make_gemv_args(a, x, x_is_f32, x_stride, m, k, weights, n, epilogue, outputs, out_stride, addend,
                                    addend_stride, rope_cos, rope_sin, head_dim, "fl_gemv_bf16");
  if (rc != FL_OK) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (epilogue) {
    case kEpiPlain: launch_gemv<kEpiPlain>(a, n / kRows, st); break;
    case kEpiF32: launch_gemv<kEpiF32>(a, n / kRows, st); break;
    case kEpiAdd: launch_gemv<kEpiAdd>(a, n / kRows, st); break;
    case kEpiSwiGlu: launch_gemv<kEpiSwiGlu>(a, n / 2, st); break;
    default: launch_gemv<kEpiRope>(a, 3 * (n / kRows), st); break;
  }
  FL_LAUNCH_CHECK("fl_gemv_bf16");
  return FL_OK;
}

extern "C" int32_t fl_gemv_bf16_chain(int32_t m, int32_t k, float eps, const uint16_t* x, const uint16_t* r,
                                      const uint16_t* w_a, const uint16_t* w_f, const uint16_t* w_b, uint16_t* h_out,
                                      int64_t stride, const uint16_t* const* weights, int32_t n, int32_t epilogue,
                                      void* const* outputs, int64_t out_stride, const uint16_t* addend,
                                      int64_t addend_stride, const uint16_t* rope_cos, const uint16_t* rope_sin,
                                      int32_t head_dim, void* stream) {
  using namespace fl;
  clear_error();
  FL_REQUIRE(r != nullptr, "fl_gemv_bf16_chain: null residual/input");
  FL_REQUIRE(k <= kChainMaxK && stride >= k && stride % 8 == 0,
             "fl_gemv_bf16_chain: K must be at most 4096 and the chain row stride a multiple of 8 >= K");
  FL_REQUIRE(x == nullptr || w_a != nullptr, "fl_gemv_bf16_chain: x needs its norm weight");
  for (const void* p : {static_cast<const void*>(x), static_cast<const void*>(r), static_cast<const void*>(w_a),
                        static_cast<const void*>(w_f), static_cast<const void*>(w_b), static_cast<const void*>(h_out)})
    FL_REQUIRE(reinterpret_cast<uintptr_t>(p) % 16 == 0, "fl_gemv_bf16_chain: every chain tensor must be 16-byte aligned");
  GemvArgs a{};
  // the GEMV's x is the chain output: its checks run on the residual row layout
  const int32_t rc = make_gemv_args(a, r, 0, stride, m, k, weights, n, epilogue, outputs, out_stride, addend,
                                    addend_stride, rope_cos, rope_sin, head_dim, "fl_gemv_bf16_chain");
  if (rc != FL_OK) return rc;
  const NormArgs c{k, eps, x, r, w_a, w_f, w_b, h_out, nullptr, stride};
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int blocks = gemv_blocks(epilogue, n);
  switch (epilogue) {
    case kEpiPlain: launch_gemv_chain<kEpiPlain>(a, c, blocks, st); break;
    case kEpiF32: launch_gemv_chain<kEpiF32>(a, c, blocks, st); break;
    case kEpiAdd: launch_gemv_chain<kEpiAdd>(a, c, blocks, st); break;
    case kEpiSwiGlu: launch_gemv_chain<kEpiSwiGlu>(a, c, blocks, st); break;
    default: launch_gemv_chain<kEpiRope>(a, c, blocks, st); break;
  }
  FL_LAUNCH_CHECK("fl_gemv_bf16_chain");
  return FL_OK;
}

extern "C" int32_t fl_norm_chain(int32_t m, int32_t d, float eps, const uint16_t* x, const uint16_t* r,
                                 const uint16_t* w_a, const uint16_t* w_f, const uint16_t* w_b, uint16_t* h_out,
                                 uint16_t* z_out, int64_t stride, void* stream) {
  using namespace fl;
  clear_error();
  FL_REQUIRE(m >= 0 && d > 0 && d % 8 == 0 && d <= kNormThreads * kNormChunks * 8 && stride >= d && stride % 8 == 0,
             "fl_norm_chain: d must be a multiple of 8 up to 8192 and the row stride a multiple of 8");
  FL_REQUIRE(r != nullptr, "fl_norm_chain: null residual/input");
  FL_REQUIRE(x == nullptr || w_a != nullptr, "fl_norm_chain: x needs its norm weight");
  FL_REQUIRE(w_b == nullptr || z_out != nullptr, "fl_norm_chain: z needs an output");
  FL_REQUIRE(h_out != nullptr || z_out != nullptr, "fl_norm_chain: nothing to write");
  for (const void* p : {static_cast<const void*>(x), static_cast<const void*>(r), static_cast<const void*>(w_a),
                        static_cast<const void*>(w_f), static_cast<const void*>(w_b),
                        static_cast<const void*>(h_out), static_cast<const void*>(z_out)})
    FL_REQUIRE(reinterpret_cast<uintptr_t>(p) % 16 == 0, "fl_norm_chain: every tensor must be 16-byte aligned");
  if (m == 0) return FL_OK;
  NormArgs a{d, eps, x, r, w_a, w_f, w_b, h_out, z_out, stride};
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (d <= kNormThreads * 8)
    hipLaunchKernelGGL(norm_chain_kernel<1>, dim3(m), dim3(kNormThreads), 0, st, a);
  else if (d <= 2 * kNormThreads * 8)
    hipLaunchKernelGGL(norm_chain_kernel<2>, dim3(m), dim3(kNormThreads), 0, st, a);
  else
    hipLaunchKernelGGL(norm_chain_kernel<kNormChunks>, dim3(m), dim3(kNormThreads), 0, st, a);
  FL_LAUNCH_CHECK("fl_norm_chain");
  return FL_OK;
}

extern "C" int32_t fl_append_tail(const fl_cache_view* view, const uint16_t* const* keys,
                                  const uint16_t* const* values, uint8_t* const* tail_active,
                                  int32_t* tail_tokens, void* stream) {
  using namespace fl;
  clear_error();
  FL_REQUIRE(view && keys && values && tail_active, "fl_append_tail: null argument");
  const fl_cache_view& v = *view;
  FL_REQUIRE(v.batch > 0 && v.heads > 0 && v.tail_capacity > 0 && v.tail_tokens, "fl_append_tail: bad view");
  FL_REQUIRE(tail_tokens == v.tail_tokens, "fl_append_tail: tail_tokens must be the view's length array");
  AppendArgs a{};
  a.v = v;
  for (int r = 0; r < 4; ++r) {
    FL_REQUIRE(keys[r] && values[r] && v.tail_key[r] && v.tail_value[r], "fl_append_tail: null row or tail");
    FL_REQUIRE(reinterpret_cast<uintptr_t>(keys[r]) % 16 == 0 && reinterpret_cast<uintptr_t>(values[r]) % 16 == 0,
               "fl_append_tail: rows must be 16-byte aligned");
    a.k[r] = keys[r];
    a.val[r] = values[r];
  }
  FL_REQUIRE(tail_active[0] && tail_active[1], "fl_append_tail: null tail_active");
  a.active[0] = tail_active[0];
  a.active[1] = tail_active[1];
  a.tail_tokens = tail_tokens;
  hipLaunchKernelGGL(append_tail_kernel, dim3(v.batch), dim3(kAppendThreads), 0, static_cast<hipStream_t>(stream), a);
  FL_LAUNCH_CHECK("fl_append_tail");
  return FL_OK;
}
