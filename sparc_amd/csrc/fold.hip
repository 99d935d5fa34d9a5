// The controls folded into an input projection (the 12-layer block stack):
// with the module input x = x_n W^T (W [width, dim], width = 2M), the control
// dot products x.u + b equal x_n (W^T u) + b, so the stack runs the controls
// over x_n with the folded directions
//   forward   f_k[d] = sum_w u_k[w] W[w, d]  (d < dim),  f_k[dim] = u_k[width]
//   backward  du_k[w] = sum_d g_k[d] W[w, d]  (w < width), du_k[width] = g_k[dim]
//             dW[w, d] += u_0[w] g_0[d] + u_1[w] g_1[d]  (optional, in place)
// for the phase (k = 0) and radial (k = 1) directions, g the gradients of the
// folded directions.  W and dW in the I/O type, everything else fp32, fp32
// arithmetic (dW rounded once, after the add).  The forward reads W once: one
// wave per block of rows, the waves' per-column sums added in LDS in wave
// order into one partial row per workgroup and direction, the partial rows
// summed in a fixed order (column_sums); the backward is one wave per
// row block, two dot products per row, and the rank-2 update of the same row
// of dW.  Replaces torch products over an fp32 copy of W, and the fp32
// rank-2 product, its cast and the add into the projection's gradient.

#include "common.h"
#include "reduce.h"
#include "sparc_hip.h"

namespace sparc {
namespace {

constexpr int kFoldMaxDim = 4096;   // 8 chunks of 64 lanes x 8 columns
constexpr int kFoldWaves = 4;       // waves per workgroup, both kernels
constexpr int kFoldRowsPerWave = 16;

constexpr int fold_nch(int64_t dim) { return dim <= 512 ? 1 : dim <= 1024 ? 2 : dim <= 2048 ? 4 : 8; }
int64_t fold_blocks(int64_t width) {
  const int64_t rows = static_cast<int64_t>(kFoldWaves) * kFoldRowsPerWave;
  return (width + rows - 1) / rows;
}

template <typename IO>
__device__ __forceinline__ void load8w(const void* base, int64_t index, float (&o)[8]) {
  if constexpr (sizeof(IO) == 2) {
    unpack<bf16, 8>(load_raw<bf16, 8>(base, index), o);
  } else {
    float a[4], b[4];
    unpack<float, 4>(load_raw<float, 4>(base, index), a);
    unpack<float, 4>(load_raw<float, 4>(base, index + 4), b);
#pragma unroll
    for (int i = 0; i < 4; ++i) { o[i] = a[i]; o[4 + i] = b[i]; }
  }
}

template <typename IO>
__device__ __forceinline__ void store8w(void* base, int64_t index, const float (&o)[8]) {
  if constexpr (sizeof(IO) == 2) {
    store_raw<bf16, 8>(base, index, pack<bf16, 8>(o));
  } else {
    const float a[4] = {o[0], o[1], o[2], o[3]}, b[4] = {o[4], o[5], o[6], o[7]};
    store_raw<float, 4>(base, index, pack<float, 4>(a));
    store_raw<float, 4>(base, index + 4, pack<float, 4>(b));
  }
}

// part [2][gridDim.x][dim]: direction k's partial row of this workgroup
template <typename IO, int NCH>
__global__ void __launch_bounds__(64 * kFoldWaves)
fold_fwd_kernel(int64_t width, int dim, const void* wt, const float* u0, const float* u1, float* part, float* f0,
                float* f1) {
  __shared__ float4 red[kFoldWaves - 1][2][2][64];  // [wave - 1][direction][half][lane]
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));  // wave-uniform
  if (blockIdx.x == 0 && threadIdx.x == 0) {  // the bias entries pass through
    f0[dim] = u0[width];
    f1[dim] = u1[width];
  }
  float a0[NCH][8], a1[NCH][8];
#pragma unroll
  for (int k = 0; k < NCH; ++k)
#pragma unroll
    for (int i = 0; i < 8; ++i) { a0[k][i] = 0.0f; a1[k][i] = 0.0f; }
  const int64_t r0 = (static_cast<int64_t>(blockIdx.x) * kFoldWaves + wave) * kFoldRowsPerWave;
  for (int j = 0; j < kFoldRowsPerWave; ++j) {
    const int64_t r = r0 + j;
    if (r >= width) break;  // wave-uniform; every wave still reaches the barriers below
    const float c0 = u0[r], c1 = u1[r];
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
      const int c = (k * 64 + lane) * 8;
      if (c < dim) {
        float w[8];
        load8w<IO>(wt, r * dim + c, w);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          a0[k][i] = fmaf(c0, w[i], a0[k][i]);
          a1[k][i] = fmaf(c1, w[i], a1[k][i]);
        }
      }
    }
  }
  float* p0 = part + static_cast<int64_t>(blockIdx.x) * dim;
  float* p1 = part + (static_cast<int64_t>(gridDim.x) + blockIdx.x) * dim;
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    if (wave > 0) {
      red[wave - 1][0][0][lane] = make_float4(a0[k][0], a0[k][1], a0[k][2], a0[k][3]);
      red[wave - 1][0][1][lane] = make_float4(a0[k][4], a0[k][5], a0[k][6], a0[k][7]);
      red[wave - 1][1][0][lane] = make_float4(a1[k][0], a1[k][1], a1[k][2], a1[k][3]);
      red[wave - 1][1][1][lane] = make_float4(a1[k][4], a1[k][5], a1[k][6], a1[k][7]);
    }
    __syncthreads();
    const int c = (k * 64 + lane) * 8;
    if (wave == 0 && c < dim) {
      float t0[8], t1[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) { t0[i] = a0[k][i]; t1[i] = a1[k][i]; }
      for (int v = 0; v < kFoldWaves - 1; ++v) {
        const float4 x0 = red[v][0][0][lane], x1 = red[v][0][1][lane];
        const float4 y0 = red[v][1][0][lane], y1 = red[v][1][1][lane];
        t0[0] += x0.x; t0[1] += x0.y; t0[2] += x0.z; t0[3] += x0.w;
        t0[4] += x1.x; t0[5] += x1.y; t0[6] += x1.z; t0[7] += x1.w;
        t1[0] += y0.x; t1[1] += y0.y; t1[2] += y0.z; t1[3] += y0.w;
        t1[4] += y1.x; t1[5] += y1.y; t1[6] += y1.z; t1[7] += y1.w;
      }
      *reinterpret_cast<float4*>(p0 + c) = make_float4(t0[0], t0[1], t0[2], t0[3]);
      *reinterpret_cast<float4*>(p0 + c + 4) = make_float4(t0[4], t0[5], t0[6], t0[7]);
      *reinterpret_cast<float4*>(p1 + c) = make_float4(t1[0], t1[1], t1[2], t1[3]);
      *reinterpret_cast<float4*>(p1 + c + 4) = make_float4(t1[4], t1[5], t1[6], t1[7]);
    }
    __syncthreads();
  }
}

// du_k[w] for the rows of this wave (and with DW, the rank-2 update of the
// same rows of dwt); one wave per kFoldRowsPerWave rows
template <typename IO, int NCH, bool DW>
__global__ void __launch_bounds__(64 * kFoldWaves)
fold_bwd_kernel(int64_t width, int dim, const void* wt, const float* u0, const float* u1, const float* g0,
                const float* g1, float* du0, float* du1, void* dwt) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  if (blockIdx.x == 0 && threadIdx.x == 0) {  // the bias entries pass through
    du0[width] = g0[dim];
    du1[width] = g1[dim];
  }
  float v0[NCH][8], v1[NCH][8];
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int c = (k * 64 + lane) * 8;
#pragma unroll
    for (int i = 0; i < 8; ++i) { v0[k][i] = 0.0f; v1[k][i] = 0.0f; }
    if (c < dim) {
#pragma unroll
      for (int i = 0; i < 8; ++i) { v0[k][i] = g0[c + i]; v1[k][i] = g1[c + i]; }
    }
  }
  const int64_t r0 = (static_cast<int64_t>(blockIdx.x) * kFoldWaves + wave) * kFoldRowsPerWave;
  for (int j = 0; j < kFoldRowsPerWave; ++j) {
    const int64_t r = r0 + j;
    if (r >= width) return;  // wave-uniform; no barrier in this kernel
    float s0 = 0.0f, s1 = 0.0f;
    const float c0 = DW ? u0[r] : 0.0f, c1 = DW ? u1[r] : 0.0f;
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
      const int c = (k * 64 + lane) * 8;
      if (c < dim) {
        float w[8], d[8];
        load8w<IO>(wt, r * dim + c, w);
        if constexpr (DW) load8w<IO>(dwt, r * dim + c, d);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          s0 = fmaf(v0[k][i], w[i], s0);
          s1 = fmaf(v1[k][i], w[i], s1);
        }
        if constexpr (DW) {
#pragma unroll
          for (int i = 0; i < 8; ++i) d[i] += fmaf(c0, v0[k][i], c1 * v1[k][i]);
          store8w<IO>(dwt, r * dim + c, d);
        }
      }
    }
    s0 = group_sum(s0, 64);
    s1 = group_sum(s1, 64);
    if (lane == 0) {
      du0[r] = s0;
      du1[r] = s1;
    }
  }
}

template <typename IO>
void launch_fold_fwd(hipStream_t st, int64_t width, int dim, const void* wt, const float* u0, const float* u1,
                     float* part, float* f0, float* f1) {
  const dim3 g(static_cast<unsigned>(fold_blocks(width))), b(64 * kFoldWaves);
  switch (fold_nch(dim)) {
    case 1: hipLaunchKernelGGL((fold_fwd_kernel<IO, 1>), g, b, 0, st, width, dim, wt, u0, u1, part, f0, f1); break;
    case 2: hipLaunchKernelGGL((fold_fwd_kernel<IO, 2>), g, b, 0, st, width, dim, wt, u0, u1, part, f0, f1); break;
    case 4: hipLaunchKernelGGL((fold_fwd_kernel<IO, 4>), g, b, 0, st, width, dim, wt, u0, u1, part, f0, f1); break;
    default: hipLaunchKernelGGL((fold_fwd_kernel<IO, 8>), g, b, 0, st, width, dim, wt, u0, u1, part, f0, f1);
  }
}
template <typename IO, bool DW>
void launch_fold_bwd(hipStream_t st, int64_t width, int dim, const void* wt, const float* u0, const float* u1,
                     const float* g0, const float* g1, float* du0, float* du1, void* dwt) {
  const dim3 g(static_cast<unsigned>(fold_blocks(width))), b(64 * kFoldWaves);
#define SPARC_FOLD_BWD(n) \
  hipLaunchKernelGGL((fold_bwd_kernel<IO, n, DW>), g, b, 0, st, width, dim, wt, u0, u1, g0, g1, du0, du1, dwt)
  switch (fold_nch(dim)) {
    case 1: SPARC_FOLD_BWD(1); break;
    case 2: SPARC_FOLD_BWD(2); break;
    case 4: SPARC_FOLD_BWD(4); break;
    default: SPARC_FOLD_BWD(8);
  }
#undef SPARC_FOLD_BWD
}

sparc_status fold_fail(sparc_status s, const char* msg) {
  snprintf(error_buffer(), 512, "%s", msg);
  return s;
}

bool fold_aligned(const void* p, size_t a) { return reinterpret_cast<uintptr_t>(p) % a == 0; }

sparc_status check_fold(int64_t width, int64_t dim, int32_t io) {
  if (width <= 0 || dim <= 0 || dim % 8 || dim > kFoldMaxDim)
    return fold_fail(SPARC_EINVAL, "controls fold: width > 0 and dim a positive multiple of 8 up to 4096 required");
  if (io != SPARC_F32 && io != SPARC_BF16) return fold_fail(SPARC_EINVAL, "controls fold: io_dtype");
  if (width > INT32_MAX || width > (int64_t(1) << 40) / dim) return fold_fail(SPARC_EINVAL, "controls fold: too large");
  return SPARC_OK;
}

sparc_status fold_hip_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) return SPARC_OK;
  snprintf(error_buffer(), 512, "%s: %s", what, hipGetErrorString(e));
  return SPARC_EHIP;
}

}  // namespace
}  // namespace sparc

// ===========================================================================
// C ABI
// ===========================================================================
extern "C" {

size_t sparc_controls_fold_workspace_bytes(int64_t width, int64_t dim) {
  using namespace sparc;
  if (width <= 0 || width > INT32_MAX || dim <= 0 || dim % 8 || dim > kFoldMaxDim) return 0;
  return static_cast<size_t>(2 * fold_blocks(width)) * static_cast<size_t>(dim) * sizeof(float) + 256;
}

sparc_status sparc_controls_fold(int64_t width, int64_t dim, int32_t io_dtype, const void* weight,
                                 const float* phase_direction, const float* radial_direction, float* folded_phase,
                                 float* folded_radial, void* workspace, size_t workspace_bytes,
                                 sparc_stream_t stream) {
  using namespace sparc;
  if (sparc_status s = check_fold(width, dim, io_dtype)) return s;
  if (!weight || !phase_direction || !radial_direction || !folded_phase || !folded_radial)
    return fold_fail(SPARC_EINVAL, "controls fold: NULL pointer");
  if (!fold_aligned(weight, 16) || !fold_aligned(workspace, 16))
    return fold_fail(SPARC_EINVAL, "controls fold: weight and the workspace must be 16-byte aligned");
  if (!workspace || workspace_bytes < sparc_controls_fold_workspace_bytes(width, dim))
    return fold_fail(SPARC_EWORKSPACE, "controls fold: workspace missing or too small");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  float* part = static_cast<float*>(workspace);
  const int D = static_cast<int>(dim);
  if (io_dtype == SPARC_BF16)
    launch_fold_fwd<sparc::bf16>(st, width, D, weight, phase_direction, radial_direction, part, folded_phase,
                                 folded_radial);
  else
    launch_fold_fwd<float>(st, width, D, weight, phase_direction, radial_direction, part, folded_phase,
                           folded_radial);
  if (sparc_status s = fold_hip_status("controls fold")) return s;
  const int64_t nb = fold_blocks(width);
  const float* in[2] = {part, part + nb * dim};
  float* out[2] = {folded_phase, folded_radial};
  return column_sums(nb, dim, 2, in, out, stream);
}

sparc_status sparc_controls_fold_backward(int64_t width, int64_t dim, int32_t io_dtype, const void* weight,
                                          const float* phase_direction, const float* radial_direction,
                                          const float* dfolded_phase, const float* dfolded_radial,
                                          float* dphase_direction, float* dradial_direction, void* dweight,
                                          sparc_stream_t stream) {
  using namespace sparc;
  if (sparc_status s = check_fold(width, dim, io_dtype)) return s;
  if (!weight || !dfolded_phase || !dfolded_radial || !dphase_direction || !dradial_direction ||
      (dweight && (!phase_direction || !radial_direction)))
    return fold_fail(SPARC_EINVAL, "controls fold backward: NULL pointer");
  if (!fold_aligned(weight, 16) || !fold_aligned(dweight, 16))
    return fold_fail(SPARC_EINVAL, "controls fold backward: weight and dweight must be 16-byte aligned");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int D = static_cast<int>(dim);
  const float *u0 = phase_direction, *u1 = radial_direction, *g0 = dfolded_phase, *g1 = dfolded_radial;
  float *du0 = dphase_direction, *du1 = dradial_direction;
  if (io_dtype == SPARC_BF16) {
    if (dweight) launch_fold_bwd<sparc::bf16, true>(st, width, D, weight, u0, u1, g0, g1, du0, du1, dweight);
    else launch_fold_bwd<sparc::bf16, false>(st, width, D, weight, u0, u1, g0, g1, du0, du1, dweight);
  } else {
    if (dweight) launch_fold_bwd<float, true>(st, width, D, weight, u0, u1, g0, g1, du0, du1, dweight);
    else launch_fold_bwd<float, false>(st, width, D, weight, u0, u1, g0, g1, du0, du1, dweight);
  }
  return fold_hip_status("controls fold backward");
}

}  // extern "C"
