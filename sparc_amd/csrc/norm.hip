// RMSNorm over the rows of a [rows, cols] matrix: the pre-norm and the final
// norm of the 12-layer block stack (torch.nn.RMSNorm's formula, which the
// stack used before):
//   forward   rstd = 1 / sqrt(mean(x^2) + eps) per row, y = (x rstd) w
//   backward  xhat = x rstd, g = dy w,
//             dx = rstd (g - xhat mean(g xhat)),  dw = sum over rows of dy xhat
// in fp32 arithmetic with x, w, y, dy, dx in the I/O type.  Forward: one wave
// per row, 8 consecutive columns per lane and chunk; backward: one wave per
// kNormBwdRows rows, and the per-column sums of dy xhat of a workgroup's
// waves form one partial row of dw; the partial rows are summed in a fixed
// order (sparc_column_sum), so dw does not depend on timing.  The reference ships
// the layer, not a network; the stack is this library's harness for the
// 12-layer training configuration.

#include "common.h"
#include "sparc_hip.h"

namespace sparc {
namespace {

constexpr int kNormWaves = 4;      // rows per forward workgroup, one per wave
constexpr int kNormMaxCols = 4096; // 8 chunks of 64 lanes x 8 columns
constexpr int kNormBwdRows = 8;    // rows per backward wave
// waves per backward workgroup (one dw partial row each): 16, fewer where a
// lane holds more columns (the register bound of 64 NW threads per workgroup)
constexpr int bwd_waves(int nch) { return nch <= 2 ? 16 : (nch <= 4 ? 8 : 4); }
constexpr int nch_of(int64_t cols) { return cols <= 512 ? 1 : cols <= 1024 ? 2 : cols <= 2048 ? 4 : 8; }
int64_t bwd_blocks(int64_t rows, int64_t cols) {
  const int64_t block_rows = static_cast<int64_t>(kNormBwdRows) * bwd_waves(nch_of(cols));
  return (rows + block_rows - 1) / block_rows;
}

template <typename IO>
__device__ __forceinline__ void load8(const void* base, int64_t index, float (&o)[8]) {
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
__device__ __forceinline__ void store8(void* base, int64_t index, const float (&v)[8]) {
  if constexpr (sizeof(IO) == 2) {
    store_raw<bf16, 8>(base, index, pack<bf16, 8>(v));
  } else {
    const float a[4] = {v[0], v[1], v[2], v[3]}, b[4] = {v[4], v[5], v[6], v[7]};
    store_raw<float, 4>(base, index, pack<float, 4>(a));
    store_raw<float, 4>(base, index + 4, pack<float, 4>(b));
  }
}

// NCH chunks of 512 columns (the last one partial when cols is not a
// multiple of 512; cols is a multiple of 8, so a lane's 8 columns are all in
// or all out)
template <typename IO, int NCH>
__global__ void __launch_bounds__(64 * kNormWaves)
rms_norm_fwd_kernel(int64_t R, int D, const void* x, const void* w, float eps, void* y, float* rstd) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kNormWaves + (threadIdx.x >> 6);
  if (row >= R) return;  // wave-uniform; nothing below synchronises the workgroup
  const int64_t base = row * D;
  float v[NCH][8];
  float ss = 0.0f;
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int c = (k * 64 + lane) * 8;
    if (c < D) {
      load8<IO>(x, base + c, v[k]);
#pragma unroll
      for (int i = 0; i < 8; ++i) ss = fmaf(v[k][i], v[k][i], ss);
    }
  }
  ss = group_sum(ss, 64);
  const float r = rsqrtf(ss / static_cast<float>(D) + eps);
  if (lane == 0) rstd[row] = r;
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int c = (k * 64 + lane) * 8;
    if (c < D) {
      float wv[8], o[8];
      load8<IO>(w, c, wv);
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = (v[k][i] * r) * wv[i];
      store8<IO>(y, base + c, o);
    }
  }
}

// kNormBwdRows rows per wave, bwd_waves(NCH) waves per workgroup; the
// waves' per-column sums of dy xhat are added in LDS in a fixed order (wave 0,
// 1, 2, ...) into one partial row per workgroup: dw_part [n_blocks, D] fp32
template <typename IO, int NCH>
__global__ void __launch_bounds__(64 * bwd_waves(NCH))
rms_norm_bwd_kernel(int64_t R, int D, const void* x, const void* w, const float* rstd, const void* dy, void* dx,
                    float* dw_part) {
  constexpr int kNormBwdWaves = bwd_waves(NCH);
  __shared__ float4 red[kNormBwdWaves - 1][2][64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));  // wave-uniform
  const int64_t r0 = (static_cast<int64_t>(blockIdx.x) * kNormBwdWaves + wave) * kNormBwdRows;
  float wv[NCH][8], acc[NCH][8];
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int c = (k * 64 + lane) * 8;
#pragma unroll
    for (int i = 0; i < 8; ++i) { wv[k][i] = 0.0f; acc[k][i] = 0.0f; }
    if (c < D) load8<IO>(w, c, wv[k]);
  }
  const float inv_d = 1.0f / static_cast<float>(D);
  // row j + 1's x and dy are loaded before row j is reduced and its dx
  // stored, so that they are in flight meanwhile (the compiler cannot move
  // them above that store itself: dx might alias x or dy)
  float xn[NCH][8] = {}, dn[NCH][8] = {};
  auto load_row = [&](int64_t row) __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
      const int c = (k * 64 + lane) * 8;
      if (c < D) {
        load8<IO>(x, row * D + c, xn[k]);
        load8<IO>(dy, row * D + c, dn[k]);
      }
    }
  };
  if (r0 < R) load_row(r0);
  for (int j = 0; j < kNormBwdRows; ++j) {
    const int64_t row = r0 + j;
    if (row >= R) break;  // wave-uniform; every wave still reaches the barriers below
    const int64_t base = row * D;
    const float r = rstd[row];
    float xv[NCH][8], dv[NCH][8];
#pragma unroll
    for (int k = 0; k < NCH; ++k)
#pragma unroll
      for (int i = 0; i < 8; ++i) { xv[k][i] = xn[k][i]; dv[k][i] = dn[k][i]; }
    if (j + 1 < kNormBwdRows && row + 1 < R) load_row(row + 1);  // wave-uniform
    float xh[NCH][8], g[NCH][8];
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
      const int c = (k * 64 + lane) * 8;
#pragma unroll
      for (int i = 0; i < 8; ++i) { xh[k][i] = 0.0f; g[k][i] = 0.0f; }
      if (c < D) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          xh[k][i] = xv[k][i] * r;
          g[k][i] = dv[k][i] * wv[k][i];
          s = fmaf(g[k][i], xh[k][i], s);
          acc[k][i] = fmaf(dv[k][i], xh[k][i], acc[k][i]);
        }
      }
    }
    const float m = group_sum(s, 64) * inv_d;  // mean(g xhat)
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
      const int c = (k * 64 + lane) * 8;
      if (c < D) {
        float o[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = r * fmaf(-xh[k][i], m, g[k][i]);
        store8<IO>(dx, base + c, o);
      }
    }
  }
  float* out = dw_part + static_cast<int64_t>(blockIdx.x) * D;
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    if (wave > 0) {
      red[wave - 1][0][lane] = make_float4(acc[k][0], acc[k][1], acc[k][2], acc[k][3]);
      red[wave - 1][1][lane] = make_float4(acc[k][4], acc[k][5], acc[k][6], acc[k][7]);
    }
    __syncthreads();
    const int c = (k * 64 + lane) * 8;
    if (wave == 0 && c < D) {
      float t[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) t[i] = acc[k][i];
      for (int v = 0; v < kNormBwdWaves - 1; ++v) {
        const float4 a = red[v][0][lane], b = red[v][1][lane];
        t[0] += a.x; t[1] += a.y; t[2] += a.z; t[3] += a.w;
        t[4] += b.x; t[5] += b.y; t[6] += b.z; t[7] += b.w;
      }
      *reinterpret_cast<float4*>(out + c) = make_float4(t[0], t[1], t[2], t[3]);
      *reinterpret_cast<float4*>(out + c + 4) = make_float4(t[4], t[5], t[6], t[7]);
    }
    __syncthreads();
  }
}

__global__ void zero_kernel(float* p, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.0f;
}

template <typename IO>
void launch_fwd(hipStream_t st, int64_t R, int D, const void* x, const void* w, float eps, void* y, float* rstd) {
  const dim3 g(static_cast<unsigned>((R + kNormWaves - 1) / kNormWaves)), b(64 * kNormWaves);
  const int nch = (D + 511) / 512;
  if (nch <= 1) hipLaunchKernelGGL((rms_norm_fwd_kernel<IO, 1>), g, b, 0, st, R, D, x, w, eps, y, rstd);
  else if (nch <= 2) hipLaunchKernelGGL((rms_norm_fwd_kernel<IO, 2>), g, b, 0, st, R, D, x, w, eps, y, rstd);
  else if (nch <= 4) hipLaunchKernelGGL((rms_norm_fwd_kernel<IO, 4>), g, b, 0, st, R, D, x, w, eps, y, rstd);
  else hipLaunchKernelGGL((rms_norm_fwd_kernel<IO, 8>), g, b, 0, st, R, D, x, w, eps, y, rstd);
}
template <typename IO>
void launch_bwd(hipStream_t st, int64_t R, int D, const void* x, const void* w, const float* rstd, const void* dy,
                void* dx, float* part) {
  const int nch = nch_of(D);
  const dim3 g(static_cast<unsigned>(bwd_blocks(R, D))), b(64 * bwd_waves(nch));
  if (nch <= 1) hipLaunchKernelGGL((rms_norm_bwd_kernel<IO, 1>), g, b, 0, st, R, D, x, w, rstd, dy, dx, part);
  else if (nch <= 2) hipLaunchKernelGGL((rms_norm_bwd_kernel<IO, 2>), g, b, 0, st, R, D, x, w, rstd, dy, dx, part);
  else if (nch <= 4) hipLaunchKernelGGL((rms_norm_bwd_kernel<IO, 4>), g, b, 0, st, R, D, x, w, rstd, dy, dx, part);
  else hipLaunchKernelGGL((rms_norm_bwd_kernel<IO, 8>), g, b, 0, st, R, D, x, w, rstd, dy, dx, part);
}

sparc_status norm_fail(sparc_status s, const char* msg) {
  snprintf(error_buffer(), 512, "%s", msg);
  return s;
}

bool aligned(const void* p, size_t a) { return reinterpret_cast<uintptr_t>(p) % a == 0; }

sparc_status check_norm(int64_t rows, int64_t cols, int32_t io) {
  if (rows < 0 || cols <= 0 || cols % 8 || cols > kNormMaxCols)
    return norm_fail(SPARC_EINVAL, "rms norm: rows >= 0 and cols a positive multiple of 8 up to 4096 required");
  if (io != SPARC_F32 && io != SPARC_BF16) return norm_fail(SPARC_EINVAL, "rms norm: io_dtype");
  // grids of rows / 4 and rows / 8 workgroups; 64-bit element offsets
  if (rows > INT32_MAX || rows > (int64_t(1) << 40) / cols) return norm_fail(SPARC_EINVAL, "rms norm: too large");
  return SPARC_OK;
}

}  // namespace
}  // namespace sparc

// ===========================================================================
// C ABI
// ===========================================================================
extern "C" {

sparc_status sparc_rms_norm_forward(int64_t rows, int64_t cols, int32_t io_dtype, const void* x, const void* weight,
                                    float eps, void* y, float* rstd, sparc_stream_t stream) {
  using namespace sparc;
  if (sparc_status s = check_norm(rows, cols, io_dtype)) return s;
  if (rows == 0) return SPARC_OK;
  if (!x || !weight || !y || !rstd) return norm_fail(SPARC_EINVAL, "rms norm forward: NULL pointer");
  if (!aligned(x, 16) || !aligned(weight, 16) || !aligned(y, 16))
    return norm_fail(SPARC_EINVAL, "rms norm forward: x, weight and y must be 16-byte aligned");
  if (!(eps >= 0.0f)) return norm_fail(SPARC_EINVAL, "rms norm forward: eps must be >= 0");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int D = static_cast<int>(cols);
  if (io_dtype == SPARC_BF16) launch_fwd<sparc::bf16>(st, rows, D, x, weight, eps, y, rstd);
  else launch_fwd<float>(st, rows, D, x, weight, eps, y, rstd);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    snprintf(error_buffer(), 512, "rms norm forward: %s", hipGetErrorString(e));
    return SPARC_EHIP;
  }
  return SPARC_OK;
}

size_t sparc_rms_norm_workspace_bytes(int64_t rows, int64_t cols) {
  using namespace sparc;
  if (rows < 0 || rows > INT32_MAX || cols <= 0 || cols % 8 || cols > kNormMaxCols) return 0;
  const int64_t blocks = bwd_blocks(rows, cols);
  return static_cast<size_t>(blocks) * static_cast<size_t>(cols) * sizeof(float) + 256;
}

sparc_status sparc_rms_norm_backward(int64_t rows, int64_t cols, int32_t io_dtype, const void* x, const void* weight,
                                     const float* rstd, const void* dy, void* dx, float* dweight, void* workspace,
                                     size_t workspace_bytes, sparc_stream_t stream) {
  using namespace sparc;
  if (sparc_status s = check_norm(rows, cols, io_dtype)) return s;
  if (!dweight) return norm_fail(SPARC_EINVAL, "rms norm backward: NULL pointer");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (rows == 0) {  // dweight is a sum over no rows (a fill kernel, not a memset: callers may capture)
    hipLaunchKernelGGL(zero_kernel, dim3(static_cast<unsigned>((cols + 255) / 256)), dim3(256), 0, st, dweight, cols);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
      snprintf(error_buffer(), 512, "rms norm backward: %s", hipGetErrorString(e));
      return SPARC_EHIP;
    }
    return SPARC_OK;
  }
  if (!x || !weight || !rstd || !dy || !dx) return norm_fail(SPARC_EINVAL, "rms norm backward: NULL pointer");
  if (!aligned(x, 16) || !aligned(weight, 16) || !aligned(dy, 16) || !aligned(dx, 16) || !aligned(workspace, 16))
    return norm_fail(SPARC_EINVAL, "rms norm backward: x, weight, dy, dx and the workspace must be 16-byte aligned");
  if (!workspace || workspace_bytes < sparc_rms_norm_workspace_bytes(rows, cols))
    return norm_fail(SPARC_EWORKSPACE, "rms norm backward: workspace missing or too small");
  const int D = static_cast<int>(cols);
  float* part = static_cast<float*>(workspace);
  if (io_dtype == SPARC_BF16) launch_bwd<sparc::bf16>(st, rows, D, x, weight, rstd, dy, dx, part);
  else launch_bwd<float>(st, rows, D, x, weight, rstd, dy, dx, part);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    snprintf(error_buffer(), 512, "rms norm backward: %s", hipGetErrorString(e));
    return SPARC_EHIP;
  }
  return sparc_column_sum(bwd_blocks(rows, cols), cols, part, dweight, 0, stream);
}

}  // extern "C"
