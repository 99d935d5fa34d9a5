// Deterministic column sums shared by the library's sources (defined in
// pointwise.hip): several sums of the same shape in one launch.
#ifndef SPARC_REDUCE_H
#define SPARC_REDUCE_H

#include <stdint.h>

#include "sparc_hip.h"

namespace sparc {

constexpr int kMaxColumnSums = 8;

// out_i[c] = sum over r < rows of in_i[r * cols + c] for i < n (n <= 8), in
// one launch (one problem per grid row), each column summed in the same
// fixed order as sparc_column_sum, so every result equals that of
// sparc_column_sum(rows, cols, in_i, out_i, 0, stream).
sparc_status column_sums(int64_t rows, int64_t cols, int n, const float* const* ins, float* const* outs,
                         sparc_stream_t stream);

}  // namespace sparc

#endif  // SPARC_REDUCE_H
