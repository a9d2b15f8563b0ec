// Work layout of the dense decode reader, shared by the reader (dense_reader.hip) and by
// the launch that merges its rows next to the loop-2 top-k (topk.hip).
#pragma once

#include "reader_common.h"

namespace fl {
namespace reader {
namespace {

// ---------------------------------------------------------------------------------
// Global work sequence.  Row bh = b*H + h contributes kTailUnits units for its BF16 tail
// (+ current token) followed by its G_b prefix groups, G_b = packed_tokens[b] / 64
// (clamped to the capacity, so a bad length cannot fault).  Wave w owns units
// [w*chunk, min((w+1)*chunk, U)), chunk = ceil(U / waves): it runs the tails whose first
// unit it owns and streams the prefix groups it owns.  Counting a tail as kTailUnits
// groups keeps the waves that also run tails from finishing last.  A wave's partial for
// row bh goes to slot w + bh: the slots of one row are contiguous and disjoint from every
// other row's.
// ---------------------------------------------------------------------------------
constexpr int kTailUnits = 3;  // measured best among 1..12 at cfg3 (contiguous-range wave partition)
constexpr int kLenCache = 1024;  // batches whose group counts are cached in LDS

__device__ __forceinline__ int row_groups(const fl_cache_view& v, int b) {
  return max(min(v.packed_tokens[b], v.token_capacity), 0) / kGroup;
}

// Group counts per batch: from LDS for the first kLenCache batches (no global load in
// the streaming loop), from the length array beyond.
struct RowLens {
  const int* lds;
  int n;
  __device__ __forceinline__ int operator()(const fl_cache_view& v, int b) const {
    return b < n ? lds[b] : row_groups(v, b);
  }
};

__device__ __forceinline__ int64_t total_units(const fl_cache_view& v, const RowLens& rl) {
  int64_t u = 0;
  for (int b = 0; b < v.batch; ++b) u += static_cast<int64_t>(v.heads) * (kTailUnits + rl(v, b));
  return u;
}

__device__ __forceinline__ int64_t chunk_of(int64_t U, int waves) { return (U + waves - 1) / waves; }

// Partials of row bh (first unit vs, gb prefix groups) under the static split in ranges
// of `chunk` units: prefix slots [f+bh, l+bh] (wave w's partial of row bh is slot w + bh)
// and the tail slot W + BH + bh.
__device__ __forceinline__ MergeParts dense_row_parts(const float* ws, int W, int BH, int bh, int64_t vs, int gb,
                                                      int64_t chunk) {
  int64_t f = 0, l = -1;
  if (gb > 0) {
    f = (vs + kTailUnits) / chunk;
    l = (vs + kTailUnits + gb - 1) / chunk;
  }
  return MergeParts{ws + (f + bh) * kPartial, static_cast<int>(l - f + 1),
                    ws + (static_cast<int64_t>(W) + BH + bh) * kPartial};
}

struct DenseMergeLds {
  int lens[kLenCache];
  MergeLdsBuf m;
};

// Merge of one row by the first kMergeThreads threads of a workgroup (every thread of
// those waves calls it).  `pieces` loops were read by one launch (dense_pair_kernel: 2):
// index p*BH + bh merges row bh of piece p, whose units follow those of the earlier
// pieces.  W: waves of the reader's grid.
__device__ __forceinline__ void dense_merge_row(DenseMergeLds& S, int index, const float* ws0, const float* ws1,
                                                int W, const fl_cache_view& v, float* out0, float* out1,
                                                int pieces) {
  for (int i = threadIdx.x; i < min(v.batch, kLenCache); i += kMergeThreads) S.lens[i] = row_groups(v, i);
  __syncthreads();
  const RowLens rl{S.lens, min(v.batch, kLenCache)};
  const int BH = v.batch * v.heads;
  const int piece = index / BH;
  const int bh = index - piece * BH;
  const float* ws = piece == 0 ? ws0 : ws1;
  float* out = piece == 0 ? out0 : out1;
  const int b = bh / v.heads, h = bh - (bh / v.heads) * v.heads;
  int64_t vs = 0, U = 0;
  for (int bb = 0; bb < v.batch; ++bb) {
    const int64_t span = static_cast<int64_t>(v.heads) * (kTailUnits + rl(v, bb));
    if (bb < b) vs += span;
    U += span;
  }
  const int gb = rl(v, b);
  vs += static_cast<int64_t>(h) * (kTailUnits + gb) + piece * U;
  const MergeParts P = dense_row_parts(ws, W, BH, bh, vs, gb, chunk_of(pieces * U, W));
  const float r = merge_softmax(P, S.m);
  if (threadIdx.x < kDim) out[static_cast<int64_t>(bh) * kDim + threadIdx.x] = r;
}

}  // namespace
}  // namespace reader
}  // namespace fl
