// J4: token-sparse update row movement and the loop-boundary token score.
//
// fl_gather_rows / fl_scatter_rows move whole rows (hidden states, K/V rows) between a
// full tensor and its compact active-row copy: index_select / index_copy_ of
// flashloop/prefill.py:158, 193-194, 237 and flashloop/engine.py:276-333.  Every
// thread moves 16 bytes when rows and strides allow it, 4 bytes otherwise; the grid
// is (row-slices, index, outer) so consecutive threads touch consecutive bytes.
//
// fl_hidden_delta_score is _hidden_delta_score (flashloop/engine.py:78-81), one wave
// per row.
#include "fl_common.h"

namespace fl {
namespace {

template <typename V, bool SCATTER>
__global__ __launch_bounds__(256) void move_rows_kernel(const uint8_t* src, int64_t s_outer, int64_t s_row,
                                                        uint8_t* dst, int64_t d_outer, int64_t d_row, int64_t rows,
                                                        int64_t row_vecs, const int32_t* index, int32_t* err) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= row_vecs) return;
  const int64_t i = blockIdx.y;
  const int64_t o = blockIdx.z;
  const int32_t t = index[i];
  if (t < 0 || t >= rows) {
    if (err && e == 0) atomicExch(err, 1);
    return;
  }
  const int64_t src_row = SCATTER ? i : t;
  const int64_t dst_row = SCATTER ? t : i;
  const V* s = reinterpret_cast<const V*>(src + o * s_outer + src_row * s_row) + e;
  V* d = reinterpret_cast<V*>(dst + o * d_outer + dst_row * d_row) + e;
  *d = *s;
}

template <bool SCATTER>
int32_t launch_move(const void* src, int64_t s_outer, int64_t s_row, void* dst, int64_t d_outer, int64_t d_row,
                    int64_t rows, int64_t outer, int64_t row_bytes, const int32_t* index, int64_t n_index,
                    int32_t* err, void* stream, const char* who) {
  FL_REQUIRE(src && dst && index, std::string(who) + ": null pointer");
  FL_REQUIRE(outer >= 0 && n_index >= 0 && rows >= 0 && row_bytes >= 0, std::string(who) + ": negative size");
  FL_REQUIRE(row_bytes % 4 == 0 && s_outer % 4 == 0 && s_row % 4 == 0 && d_outer % 4 == 0 && d_row % 4 == 0,
             std::string(who) + ": row bytes and strides must be multiples of 4");
  FL_REQUIRE(reinterpret_cast<uintptr_t>(src) % 4 == 0 && reinterpret_cast<uintptr_t>(dst) % 4 == 0,
             std::string(who) + ": pointers must be 4-byte aligned");
  FL_REQUIRE(n_index <= 65535 * 1024LL && outer <= 65535, std::string(who) + ": grid too large");
  if (outer == 0 || n_index == 0 || row_bytes == 0) return FL_OK;
  const bool vec16 = row_bytes % 16 == 0 && s_outer % 16 == 0 && s_row % 16 == 0 && d_outer % 16 == 0 &&
                     d_row % 16 == 0 && reinterpret_cast<uintptr_t>(src) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(dst) % 16 == 0;
  const int64_t vecs = vec16 ? row_bytes / 16 : row_bytes / 4;
  const dim3 grid(static_cast<unsigned>((vecs + 255) / 256), static_cast<unsigned>(n_index),
                  static_cast<unsigned>(outer));
  FL_REQUIRE(n_index <= 2147483647LL, std::string(who) + ": too many indices");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint8_t* s = static_cast<const uint8_t*>(src);
  uint8_t* d = static_cast<uint8_t*>(dst);
  if (vec16)
    hipLaunchKernelGGL((move_rows_kernel<uint4, SCATTER>), grid, dim3(256), 0, st, s, s_outer, s_row, d, d_outer,
                       d_row, rows, vecs, index, err);
  else
    hipLaunchKernelGGL((move_rows_kernel<uint32_t, SCATTER>), grid, dim3(256), 0, st, s, s_outer, s_row, d, d_outer,
                       d_row, rows, vecs, index, err);
  FL_LAUNCH_CHECK(who);
  return FL_OK;
}

__global__ __launch_bounds__(256) void hidden_delta_score_kernel(const uint16_t* cur, const uint16_t* prev,
                                                                 int64_t rows, int dim, float* score) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int lane = threadIdx.x & 63;
  const uint16_t* c = cur + r * dim;
  const uint16_t* p = prev + r * dim;
  float num = 0.0f, den = 0.0f;
  for (int i = lane; i < dim; i += kWave) {
    const float a = bf16_to_f32(c[i]);
    const float d = a - bf16_to_f32(p[i]);
    num = fmaf(d, d, num);
    den = fmaf(a, a, den);
  }
  num = wave_sum(num);
  den = wave_sum(den);
  if (lane == 0) score[r] = sqrtf(num) / fmaxf(sqrtf(den), 1e-12f);
}

}  // namespace
}  // namespace fl

extern "C" int32_t fl_gather_rows(const void* src, int64_t src_outer_stride, int64_t src_row_stride, int64_t src_rows,
                                  void* dst, int64_t dst_outer_stride, int64_t dst_row_stride, int64_t outer,
                                  int64_t row_bytes, const int32_t* index, int64_t n_index, int32_t* error_flag,
                                  void* stream) {
  fl::clear_error();
  return fl::launch_move<false>(src, src_outer_stride, src_row_stride, dst, dst_outer_stride, dst_row_stride,
                                src_rows, outer, row_bytes, index, n_index, error_flag, stream, "fl_gather_rows");
}

extern "C" int32_t fl_scatter_rows(const void* src, int64_t src_outer_stride, int64_t src_row_stride, void* dst,
                                   int64_t dst_outer_stride, int64_t dst_row_stride, int64_t dst_rows, int64_t outer,
                                   int64_t row_bytes, const int32_t* index, int64_t n_index, int32_t* error_flag,
                                   void* stream) {
  fl::clear_error();
  return fl::launch_move<true>(src, src_outer_stride, src_row_stride, dst, dst_outer_stride, dst_row_stride,
                               dst_rows, outer, row_bytes, index, n_index, error_flag, stream, "fl_scatter_rows");
}

extern "C" int32_t fl_hidden_delta_score(const uint16_t* cur, const uint16_t* prev, int64_t rows, int32_t dim,
                                         float* score, void* stream) {
  using namespace fl;
  clear_error();
  FL_REQUIRE(cur && prev && score, "fl_hidden_delta_score: null pointer");
  FL_REQUIRE(rows >= 0 && dim > 0, "fl_hidden_delta_score: bad shape");
  if (rows == 0) return FL_OK;
  hipLaunchKernelGGL(hidden_delta_score_kernel, dim3(static_cast<unsigned>((rows + 3) / 4)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), cur, prev, rows, dim, score);
  FL_LAUNCH_CHECK("fl_hidden_delta_score");
  return FL_OK;
}
