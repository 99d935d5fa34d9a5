// The P1 scan of sparc_scan_forward / sparc_scan_backward with one gate pair
// (eta, delta) per token, run on the one-wave-per-chain kernels of the fused
// module path (mixer.hip) with the writes given instead of computed from x;
// and the carry across time segments that the serial scan kernels share with
// them.  Declared here for scan.hip (the C ABI), defined in mixer.hip.
#ifndef SPARC_P1_FUSED_H
#define SPARC_P1_FUSED_H

#include <stddef.h>
#include <stdint.h>

#include "sparc_hip.h"

namespace sparc {

// Whether a descriptor can take these kernels: P1, G = 1, no forced
// algorithm, M a multiple of 4, sizes within the kernels' limits (segment
// resets and reset_first included).  Pointer alignment is checked by the
// caller.
bool p1_fused_shape(const sparc_scan_desc* d);

// Workspace bytes of p1_fused_forward (direction 0) / _backward (1).
size_t p1_fused_workspace_bytes(const sparc_scan_desc* d, int direction);

// Forward: y_re, y_im [B,T,M] the states (or, with SPARC_FLAG_RELU_OUTPUT,
// y_re = relu(cat(h_re, h_im)) [B,T,2M]) and the chunk states
// [B][ceil(T/64)][M][2], as sparc_scan_forward.  T > 0.
sparc_status p1_fused_forward(const sparc_scan_desc* d, const float* eta, const float* delta,
                              const float* nu_log, const float* theta_log, const void* w_re, const void* w_im,
                              const float* h0_re, const float* h0_im, const int32_t* segment_pos, void* y_re,
                              void* y_im, float* chunk_state, void* workspace, size_t workspace_bytes,
                              sparc_stream_t stream);

// Backward from the forward's states y_re, y_im (no relu output).  T > 0.
sparc_status p1_fused_backward(const sparc_scan_desc* d, const float* eta, const float* delta,
                               const float* nu_log, const float* theta_log, const void* y_re, const void* y_im,
                               const float* h0_re, const float* h0_im, const int32_t* segment_pos,
                               const void* dy_re, const void* dy_im, const float* dlast_re, const float* dlast_im,
                               void* dw_re, void* dw_im, float* deta, float* ddelta, float* dnu_log,
                               float* dtheta_log, float* dh0_re, float* dh0_im, void* workspace,
                               size_t workspace_bytes, sparc_stream_t stream);

// The carry across time segments of the scan kernels (mixer.hip's
// mixer_seg_carry_kernel): from each segment's map (P, Q) in seg_sum
// [B][n_seg][M][4], the state (reverse = 0, from init = h0 or zero) or the
// adjoint (reverse = 1, from init = dlast or zero) entering every segment,
// into seg_state [B][n_seg][M][2].  Real scans pass maps with zero imaginary
// parts and init_im = NULL.  Launch errors are left for the caller's
// hipGetLastError.
sparc_status seg_carry(int64_t B, int64_t M, int n_seg, int reverse, const float* seg_sum, const float* init_re,
                       const float* init_im, float* seg_state, sparc_stream_t stream);

}  // namespace sparc

#endif  // SPARC_P1_FUSED_H
