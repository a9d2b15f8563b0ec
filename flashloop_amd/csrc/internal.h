// Host-side entry points shared between the library's translation units (not exported).
#pragma once

#include "fl_common.h"

namespace fl {
// Top-k of a dense read's logits and the merge of its rows, in one launch (topk.hip).
int32_t launch_select_merge(const fl_cache_view& v, const float* ws, int W, float* out, const float* logits,
                            int64_t logits_stride, double fraction, int32_t capacity, int32_t* indices,
                            uint8_t* valid, float* mass, float* weights, int32_t* counts, int32_t* nonfinite,
                            hipStream_t st);
// Whether launch_select_merge takes rows of this stride at this fraction (the register-
// resident top-k: at most 35840 keys, at most 8192 selected).
bool select_merge_fits(int64_t logits_stride, double fraction);
}  // namespace fl
