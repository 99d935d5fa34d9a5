// SPARC mixer sequence path for gfx950: the drop-in module's forward and
// backward with the P1 controls, the gain*tanh write, the scan and the
// relu(cat) epilogue fused, reading x directly.
//
// Forward (sparc_mixer_forward):
//   1. mixer_prepare_kernel: per-mode constants (nu, e^{i theta}, gain, ...).
//   2. ctrl_fwd_kernel: eta, delta per token (two dot products over the 2M
//      inputs, tanh).
//   3. mixer_fwd_kernel: one wave per chain (batch row, block of 64*V modes)
//      walks T in order: per step and mode the P1 transition, the write
//      gain*tanh(x) and h <- a h + w in fp32, stores y = relu(cat(h_re, h_im))
//      and the state h in the I/O dtype (saved for the backward, as the
//      reference saves out_r / out_i).
// Backward (sparc_mixer_backward):
//   4. mixer_bwd_kernel: one wave per chain in reverse time: the adjoint
//      lambda_t = mask_t dy_t + conj(a_{t+1}) lambda_{t+1}, the write path's
//      dx and the per-mode parameter gradients (in registers); each step's
//      per-lane contributions to d eta_t and d delta_t are summed over the
//      lanes in the wave (reduce-scatter) into one partial per (token, mode
//      block).
//   5. deterministic column sums: per token over the mode blocks, per mode
//      over the batch rows.
//   6. ctrl_bwd_kernel: dx += d p0_t * u_phase + d p1_t * u_radial (the
//      controls' input gradient) in place, and the direction gradients as
//      partial sums over row blocks.
// sparc_mixer_scan_forward / _backward run 1 + 3 / 4 + 5 (the controls are
// the caller's); sparc_controls_forward / _backward run 2 / 6 alone over rows
// of any width that is a multiple of 8.
// The P1 scan of sparc_scan_forward / _backward with one (eta, delta) per
// token runs 1 + 3 / 4 + 5 in another chain mode (p1_fused.h): the writes
// given instead of x, the states (or relu(cat)) and the chunk states out,
// reset steps; backward dw instead of dx and the transition gradients only.
// Few chains split time into segments (summary pass, carry, replay) in
// every mode.
//
// Reference replaced: make_controls / make_scan_inputs / _latest_write_forward
// (sparc-kernal/forward/control.py:129-195), _SPARCChunkScan forward and
// backward (sparc-kernal/backward/scan.py:1126-1640) and, with resets,
// _SPARCTiledSerialScan (:971-1070), the output epilogue
// (sparc-kernal/forward/scan.py:1598-1603), _latest_write_backward and
// _LatestSPARCWrite (sparc-kernal/backward/control.py:10-137).

#include <stdarg.h>
#include <stdio.h>

#include <atomic>
#include <mutex>
#include <type_traits>

#include "common.h"
#include "p1_fused.h"
#include "reduce.h"
#include "sparc_hip.h"

namespace sparc {
namespace mix {

constexpr float kLog16 = 2.772588722239781f;
constexpr float kInvLog16 = 0.36067376022224085f;
constexpr float kHalfPi = 1.5707963267948966f;
constexpr float kTwoOverPi = 0.6366197723675814f;
constexpr int kConsts = 12;    // floats per mode in the constants table
constexpr float kLog2e = 1.4426950408889634f;
#ifndef SPARC_MIXER_FWD_S
#define SPARC_MIXER_FWD_S 8
#endif
constexpr int kS = SPARC_MIXER_FWD_S;  // steps per prefetched block of the forward scan
constexpr int kCtrlRows = 16;  // rows per workgroup of the controls forward
constexpr int kCtrlBwdRows = 128;  // rows per workgroup of the controls backward
constexpr int kMaxRowBlocks = 65535;  // grid.y limit: more row blocks loop in the workgroups
// bf16 x: the write is rounded to bf16 before the scan, as the reference
// stores it in x's dtype (write_r.to(x.dtype), sparc-kernal/forward/
// control.py:162-163), and its gradient reaches the write's backward rounded
// to bf16 (the scan returns grad_br in the writes' dtype); the transition
// gradients keep the fp32 adjoint, as inside the reference's scan kernel.
#ifndef SPARC_MIXER_ROUND_WRITE
#define SPARC_MIXER_ROUND_WRITE 1
#endif
template <typename IO> constexpr bool kRoundWrite = SPARC_MIXER_ROUND_WRITE && sizeof(IO) == 2;

// What a chain of the scan kernels reads and writes.
//   kModule: x in (the write is gain * tanh x); y = relu(cat(h_re, h_im))
//            and the saved states h_re, h_im out; backward dx out.
//   kPlanes: the writes w_re, w_im in; the states y_re, y_im (through h_re,
//            h_im) and the chunk states out; backward dw out (the P1 scan of
//            sparc_scan_forward / _backward with one gate pair per token).
//   kRelu:   as kPlanes, but y = relu(cat(h_re, h_im)) out instead of the
//            states (forward only).
//   | kReset: kPlanes or kRelu with reset steps (segment_pos[b, t] == 0, or
//            step 0 with reset_first): the transition there is 0.
//   | kCoop: the module backward in one launch that also runs the controls'
//            backward (dx completed, direction gradients): see
//            mixer_bwd_kernel.
enum : int { kModule = 0, kPlanes = 1, kRelu = 2, kReset = 4, kCoop = 8 };
constexpr int kStateChunk = 64;  // steps per saved chunk state (sparc_scan_chunk_length)
// A lane byte offset past every buffer resource of these kernels (each spans
// less than 2^31 bytes): the hardware range check drops a store through it.
// Lanes that must not store (past M) store through it, so that no store
// sits under a branch: a branch per step splits the block's straight-line
// code, and the compiler's wait for the prefetched loads then also covers
// every store issued before them (the path that skips the stores has fewer
// memory operations in flight).
constexpr uint32_t kDropOffset = 0x80000000u;

struct Args {
  int B, T, M, n_mb;
  const void* x;
  const float* consts;
  const float* eta;
  const float* delta;
  void* y;
  void* h_re;
  void* h_im;
  float* last_re;
  float* last_im;
  // backward
  const void* dy;
  const float* dlast_re;
  const float* dlast_im;
  void* dx;
  float* part_tok;   // [2][n_mb][B*T]: d eta, d delta partials per mode block
  float* part_mode;  // [5][B*n_seg][M]: nu_log, theta_log, write_log_gain, write_phase_response, write_radial_response
  // time segments: the chains of segment s cover steps [s*t_seg, min(T, (s+1)*t_seg));
  // a launch runs segments seg_lo, seg_lo+1, ... (grid = B * n_mb * segments)
  int n_seg, t_seg, seg_lo;
  float* seg_sum;    // [B][n_seg][M][4]: each segment's map (P, Q): h_out = P h_in + Q (complex)
  float* seg_state;  // [B][n_seg][M][2]: the state (forward) or adjoint (backward) entering each segment
  // backward in time pieces (segments without the summary pass): one launch
  // per piece, the last first; a piece leaves the adjoint entering the piece
  // before it in seg_state, the last piece starts from dlast; piece s keeps
  // its per-token partials in part_tok + s*2*n_mb*B*t_seg as [2][n_mb][B][t_seg]
  int piped;
  // kPlanes / kRelu: the writes (forward) or their gradients (backward,
  // through dy = dy_re and dx = dw_re), [B,T,M] each; the initial state and
  // its gradient [B,M] fp32 (NULL: zero / not wanted); the chunk states
  // [B][ceil(T/64)][M][2] fp32
  const void* w_re;
  const void* w_im;
  const void* dy_im;
  void* dw_im;
  const float* h0_re;
  const float* h0_im;
  float* dh0_re;
  float* dh0_im;
  float* chunk_state;
  const int32_t* segpos;  // [B,T] or NULL (kReset)
  int reset_first;        // kReset without segpos: step 0 resets
  // kCoop: the directions [2M + 1] (phase, radial); the error word; every
  // chain's wave sums of every block [B*n_blk][n_mb][2 kS] and the blocks'
  // controls gradients [B*n_blk][2 kS] (both kCoopEmpty at launch), the same
  // gradients per token [2][B*T] (phase, radial projection); the direction
  // gradients per batch row [2][B][2M]; blocks per chain; polls before a
  // wait gives up
  const float* pdir;
  const float* rdir;
  uint32_t* coop_error;
  float* coop_part;
  float* coop_sum;
  float* coop_dtok;
  float* coop_pd;
  int coop_nblk;
  uint32_t coop_spin;
};

// kCoop ring entry (LDS): one step's dx of one mode, rounded to the I/O type
// (the value the controls' backward adds its rank-2 term to), and its x.
template <typename IO> struct CoopRing;
template <> struct CoopRing<bf16> {
  using T = uint2;  // bf16 pairs, re in the low half: dx, x
  static __device__ __forceinline__ T put(float dr, float di, uint16_t xr, uint16_t xi) {
    return make_uint2(pack_bf16x2(dr, di), static_cast<uint32_t>(xr) | (static_cast<uint32_t>(xi) << 16));
  }
  static __device__ __forceinline__ void get(const T& v, float& dr, float& di, float& xr, float& xi) {
    dr = __uint_as_float(v.x << 16);
    di = __uint_as_float(v.x & 0xffff0000u);
    xr = __uint_as_float(v.y << 16);
    xi = __uint_as_float(v.y & 0xffff0000u);
  }
};
template <> struct CoopRing<float> {
  using T = float4;  // dx re, dx im, x re, x im
  static __device__ __forceinline__ T put(float dr, float di, float xr, float xi) { return make_float4(dr, di, xr, xi); }
  static __device__ __forceinline__ void get(const T& v, float& dr, float& di, float& xr, float& xi) {
    dr = v.x;
    di = v.y;
    xr = v.z;
    xi = v.w;
  }
};
// Blocks a chain keeps before completing them (its ring slots, 16 KB of LDS
// per wave): a block's controls gradient is ready about two blocks after the
// block (the records stored at its end, reduced at a later block's end);
// the rest absorbs the chains' skew.
template <typename IO> constexpr int kCoopLag = sizeof(IO) == 2 ? 8 : 4;
// The records and the blocks' controls gradients start as this value, a
// signalling NaN (arithmetic quiets those, so no computed value has this bit
// pattern): a value that differs from it is final.
constexpr uint32_t kCoopEmpty = 0x7fa00001u;

// kReset: whether step t of batch row b keeps its transition (1) or resets
// (0).  segment_pos is read through a buffer resource that is empty without
// it (no load under a branch); segment_pos wins over reset_first.
__device__ __forceinline__ int p1_keep(const Args& a, int b, int t) {
  const bool sp = a.segpos != nullptr;
  const __amdgpu_buffer_rsrc_t r =
      make_rsrc(sp ? static_cast<const void*>(a.segpos + static_cast<int64_t>(b) * a.T) : a.consts, sp ? a.T * 4u : 0u);
  const int v = static_cast<int>(__builtin_amdgcn_raw_buffer_load_b32(r, static_cast<uint32_t>(t) * 4u, 0, CPOL_DEFAULT));
  return sp ? (v != 0) : !(a.reset_first && t == 0);
}

// Chain index of this workgroup -> (batch row, mode block, segment, steps).
struct ChainPos {
  int b, mb, seg, t_begin, t_end;
};
__device__ __forceinline__ ChainPos chain_pos(const Args& a) {
  const int idx = xcd_swizzle(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x));
  const int n_chains = a.B * a.n_mb;
  const int sj = idx / n_chains, chain = idx - sj * n_chains;
  ChainPos c;
  c.b = chain / a.n_mb;
  c.mb = chain - c.b * a.n_mb;
  c.seg = a.seg_lo + sj;
  c.t_begin = c.seg * a.t_seg;
  c.t_end = min(a.T, c.t_begin + a.t_seg);
  return c;
}

// Per-mode constants, folded so that the per-step arithmetic is short:
//   c0 = (nu, cos theta, sin theta, g2 = 4 gamma^2 / expm1(-2 nu))
//        gain = sqrt(g2 * em (2 + em)) * sigmoid(q), em = expm1(-nu e^eta)
//        (= gamma * sqrt(expm1(-2 nu e^eta) / expm1(-2 nu)) * 2 sigmoid(q))
//   c1 = (pl, rl, theta, kappa): -q log2(e) = delta * pl + eta * rl with
//        pl = -wpr log2(e) 2/pi, rl = -wrr log2(e) / log16;
//        kappa = nu e^{-2 nu} / (1 - e^{-2 nu})
//   c2 = (wrr / log16, wpr 2/pi, 0, 0)
// With no write parameters (wlg NULL: the P1 scan with the writes given) the
// write constants are those of gamma = 1, wpr = wrr = 0, which nothing reads.
__global__ void __launch_bounds__(256)
mixer_prepare_kernel(int M, const float* nu_log, const float* theta_log, const float* wlg,
                     const float* wpr, const float* wrr, float* consts) {
  const int m = blockIdx.x * 256 + threadIdx.x;
  if (m >= M) return;
  const float nu = expf(nu_log[m]);
  float sn, cs;
  const float theta = theta_rotation(theta_log[m], cs, sn);
  const bool wp = wlg != nullptr;
  const float gam = wp ? expf(wlg[m]) : 1.0f, pr = wp ? wpr[m] : 0.0f, rr = wp ? wrr[m] : 0.0f;
  const float cinv = 1.0f / expm1f(-2.0f * nu);
  float4* c = reinterpret_cast<float4*>(consts + static_cast<int64_t>(m) * kConsts);
  c[0] = make_float4(nu, cs, sn, 4.0f * gam * gam * cinv);
  c[1] = make_float4(-pr * kLog2e * kTwoOverPi, -rr * kLog2e * kInvLog16, theta, -nu * (1.0f + cinv));
  c[2] = make_float4(rr * kInvLog16, pr * kTwoOverPi, 0.0f, 0.0f);
}

// ---------------------------------------------------------------------------
// controls forward: eta = log16 tanh(x.u_r + b_r), delta = pi/2 tanh(x.u_p + b_p)
// ---------------------------------------------------------------------------
// A workgroup of NW waves takes kCtrlRows rows; each thread 8 consecutive
// inputs per pass, the direction values it loads serving every row of the
// workgroup.  One wave for rows of up to 1024 inputs (no idle waves in the
// reduction), four above.
template <typename IO, int NW>
__global__ void __launch_bounds__(NW * 64)
ctrl_fwd_kernel(int64_t R, int W, const void* x, const float* pdir, const float* rdir,
                float* eta, float* delta) {
  __shared__ float red[NW][2 * kCtrlRows];
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * kCtrlRows;
  float acc[2 * kCtrlRows];
#pragma unroll
  for (int i = 0; i < 2 * kCtrlRows; ++i) acc[i] = 0.0f;
  for (int c = threadIdx.x * 8; c < W; c += NW * 64 * 8) {
    float u0[8], u1[8];
    *reinterpret_cast<float4*>(u0) = *reinterpret_cast<const float4*>(pdir + c);
    *reinterpret_cast<float4*>(u0 + 4) = *reinterpret_cast<const float4*>(pdir + c + 4);
    *reinterpret_cast<float4*>(u1) = *reinterpret_cast<const float4*>(rdir + c);
    *reinterpret_cast<float4*>(u1 + 4) = *reinterpret_cast<const float4*>(rdir + c + 4);
#pragma unroll
    for (int r = 0; r < kCtrlRows; ++r) {
      const int64_t row = r0 + r < R ? r0 + r : R - 1;  // rows past R repeat the last, unused
      float xv[8];
      if constexpr (sizeof(IO) == 2) {
        unpack<bf16, 8>(load_raw_nt<bf16, 8>(x, row * W + c), xv);
      } else {
        float a[4], b[4];
        unpack<float, 4>(load_raw_nt<float, 4>(x, row * W + c), a);
        unpack<float, 4>(load_raw_nt<float, 4>(x, row * W + c + 4), b);
#pragma unroll
        for (int i = 0; i < 4; ++i) { xv[i] = a[i]; xv[4 + i] = b[i]; }
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        acc[2 * r] = fmaf(xv[i], u0[i], acc[2 * r]);
        acc[2 * r + 1] = fmaf(xv[i], u1[i], acc[2 * r + 1]);
      }
    }
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  static_assert(2 * kCtrlRows == 32, "two sums per leader lane below");
  wave_sums_to_leaders<2 * kCtrlRows>(acc);  // lanes 4k: the sums of values 2k, 2k + 1
  if (lane % 4 == 0) {
    red[wave][lane / 2] = acc[0];
    red[wave][lane / 2 + 1] = acc[1];
  }
  __syncthreads();
  if (threadIdx.x < kCtrlRows) {
    const int r = threadIdx.x;
    if (r0 + r < R) {
      float p0 = pdir[W], p1 = rdir[W];  // the bias entries
#pragma unroll
      for (int w = 0; w < NW; ++w) { p0 += red[w][2 * r]; p1 += red[w][2 * r + 1]; }
      eta[r0 + r] = kLog16 * tanhf(p1);
      delta[r0 + r] = kHalfPi * tanhf(p0);
    }
  }
}

template <typename IO>
void launch_ctrl_fwd(hipStream_t st, int64_t R, int W, const void* x, const float* pdir, const float* rdir,
                     float* eta, float* delta) {
  const dim3 g(static_cast<unsigned>((R + kCtrlRows - 1) / kCtrlRows));
  if (W <= 1024)
    hipLaunchKernelGGL((ctrl_fwd_kernel<IO, 1>), g, dim3(64), 0, st, R, W, x, pdir, rdir, eta, delta);
  else
    hipLaunchKernelGGL((ctrl_fwd_kernel<IO, 4>), g, dim3(256), 0, st, R, W, x, pdir, rdir, eta, delta);
}

// ---------------------------------------------------------------------------
// per-mode constants of a lane's V modes
// ---------------------------------------------------------------------------
template <int V, bool BWD>
struct ModeConsts {
  float nu[V], nul[V], ct[V], st[V], g2[V], pl[V], rl[V], th[V], kappa[V], wrr_s[V], wpr_s[V];
  __device__ __forceinline__ void load(const float* consts, int m0, bool ok) {
#pragma unroll
    for (int v = 0; v < V; ++v) {
      // lanes past M get zero constants: their transition is 0, their gain
      // and every per-token contribution 0 (finite inputs give finite zeros)
      const int m = ok ? m0 + v : 0;
      const float* c = consts + static_cast<int64_t>(m) * kConsts;
      const float4 c0 = *reinterpret_cast<const float4*>(c);
      const float4 c1 = *reinterpret_cast<const float4*>(c + 4);
      nu[v] = ok ? c0.x : 0.0f; ct[v] = ok ? c0.y : 0.0f; st[v] = ok ? c0.z : 0.0f; g2[v] = ok ? c0.w : 0.0f;
      pl[v] = ok ? c1.x : 0.0f; rl[v] = ok ? c1.y : 0.0f; th[v] = ok ? c1.z : 0.0f; kappa[v] = ok ? c1.w : 0.0f;
      nul[v] = nu[v] * kLog2e;
      if constexpr (BWD) {
        const float4 c2 = *reinterpret_cast<const float4*>(c + 8);
        wrr_s[v] = ok ? c2.x : 0.0f; wpr_s[v] = ok ? c2.y : 0.0f;
      }
    }
  }
};

// How the kernels of one I/O type and chain mode evaluate the P1 transition
// (every kernel of the pair the same way, so that forward, backward and the
// summary passes of time segments see the same a):
//   HW   (bf16 I/O): the sine and cosine of the phase step from the hardware
//        (sincos_rev_hw) instead of the degree-9/10 polynomials;
//   FAST (bf16 I/O, writes given): rho = 2^{-nu log2(e) E} and em = rho - 1
//        from the hardware exponential alone, without expm1's series for
//        |nu E| < 1/16.  em then carries the exponential's absolute error
//        (~6e-8, the size of rho's own fp32 rounding) rather than a relative
//        one; with the writes given, em only turns the phase (by em delta)
//        and weighs the d delta terms, where that error is below the fp32
//        rounding of rho.  The module keeps the series: its write gain goes
//        as sqrt(em) for slow modes.
// fp32 I/O keeps the polynomials and the series.
template <typename IO, int MODE>
struct P1Math {
  static constexpr bool HW = sizeof(IO) == 2;
  static constexpr bool FAST = HW && (MODE & 3) != kModule;
};

// The P1 transitions of a block of S steps for the lane's V modes, from each
// step's E = e^eta, delta and (HW) dr = -delta / (2 pi), written one level at
// a time across the S*V values so that their dependency chains interleave.
// a = rho e^{i (theta + (1 - rho) delta)}, rho = exp(-nu E), with rho - 1
// (em) formed as P1Math says; the value of p1_step, value for value.
template <typename IO, int MODE, int S, int V, bool BWD>
__device__ __forceinline__ void p1_block_transitions(const ModeConsts<V, BWD>& mc, const float (&E)[S],
                                                     const float (&dl)[S], const float (&dr)[S],
                                                     float (&ar)[S][V], float (&ai)[S][V],
                                                     float (&em_out)[S][V]) {
  using PM = P1Math<IO, MODE>;
  constexpr int N = S * V;
  float q[N], em[N], rho[N], su[N], cu[N];
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int v = 0; v < V; ++v) q[s * V + v] = PM::FAST ? -mc.nul[v] * E[s] : -mc.nu[v] * E[s];
  if constexpr (PM::FAST) {
#pragma unroll
    for (int i = 0; i < N; ++i) rho[i] = __builtin_amdgcn_exp2f(q[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) em[i] = rho[i] - 1.0f;
  } else {
    expm1_nonpos_n<N>(q, em);
#pragma unroll
    for (int i = 0; i < N; ++i) rho[i] = 1.0f + em[i];
  }
  if constexpr (PM::HW) {
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int v = 0; v < V; ++v) sincos_rev_hw(em[s * V + v] * dr[s], su[s * V + v], cu[s * V + v]);
  } else {
    float u[N];
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int v = 0; v < V; ++v) u[s * V + v] = -em[s * V + v] * dl[s];
    sincos_half_n<N>(u, su, cu);
  }
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int i = s * V + v;
      ar[s][v] = rho[i] * fmaf(mc.ct[v], cu[i], -mc.st[v] * su[i]);
      ai[s][v] = rho[i] * fmaf(mc.st[v], cu[i], mc.ct[v] * su[i]);
      em_out[s][v] = em[i];
    }
}

// The block's per-step values from lanes s of ee (e^eta), dv (delta), as
// read by p1_block_transitions.
template <int S>
__device__ __forceinline__ void p1_block_steps(float ee, float dv, float (&E)[S], float (&dl)[S], float (&dr)[S]) {
  const float drv = dv * kNegInv2Pi;
#pragma unroll
  for (int s = 0; s < S; ++s) {
    E[s] = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(ee), s));
    dl[s] = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(dv), s));
    dr[s] = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(drv), s));
  }
}

// Reset steps of a block (lane s of kv: 0 where step s resets): a := 0.  The
// transition gradients at such a step then vanish with it, and so does the
// adjoint carried past it.
template <int S, int V>
__device__ __forceinline__ void p1_block_resets(int kv, float (&ar)[S][V], float (&ai)[S][V]) {
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const bool keep = __builtin_amdgcn_readlane(kv, s) != 0;  // wave-uniform
#pragma unroll
    for (int v = 0; v < V; ++v) {
      ar[s][v] = keep ? ar[s][v] : 0.0f;
      ai[s][v] = keep ? ai[s][v] : 0.0f;
    }
  }
}

// Per-step values of the P1 transition and write of one mode.
struct StepMode {
  float em, rho, ar, ai, gain, sg;
};
// HW: the phase step's sine and cosine from the hardware (P1Math), dr =
// -delta / (2 pi).
template <bool HW>
__device__ __forceinline__ StepMode p1_step(float nu, float ct, float st, float g2, float pl, float rl,
                                             float E, float eta, float delta, float dr) {
  StepMode o;
  o.em = expm1_nonpos(-nu * E);  // rho - 1
  o.rho = 1.0f + o.em;
  float su, cu;
  if constexpr (HW) sincos_rev_hw(o.em * dr, su, cu);
  else sincos_half(-o.em * delta, su, cu);  // phase (1 - rho) delta, |.| <= pi/2
  o.ar = o.rho * fmaf(ct, cu, -st * su);
  o.ai = o.rho * fmaf(st, cu, ct * su);
  // em (2 + em) = expm1(-2 nu E)
  o.sg = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(fmaf(delta, pl, eta * rl)));  // sigmoid(q)
  o.gain = __builtin_amdgcn_sqrtf(g2 * fmaf(o.em, o.em, o.em + o.em)) * o.sg;
  return o;
}

// ---------------------------------------------------------------------------
// forward scan: one wave per chain
// ---------------------------------------------------------------------------
// Plane loads are unconditional with clamped addresses (steps past T re-read
// row T-1; lanes past M read their block's first element) and the next
// block is always prefetched (the last block re-reads itself), so that the
// wait before a block never covers the prefetch of the next one.
template <typename IO, int V, bool SUMMARY, int MODE>
__global__ void __launch_bounds__(64, 1)
mixer_fwd_kernel(Args a) {
  using RawT = typename Raw<IO, V>::T;
  constexpr int ESZ = sizeof(IO);
  constexpr int MB = 64 * V;
  constexpr int CM = MODE & 3;             // the chain mode without kReset
  constexpr bool RST = (MODE & kReset) != 0;
  constexpr bool GW = CM != kModule;  // the writes are given
  static_assert(kStateChunk % kS == 0, "blocks must tile the saved-state chunks");
  static_assert(GW || !RST, "resets in the P1 scan only");
  // a summary's loads keep their lines in the caches (the replay that follows
  // reads the same rows again); the replay's loads are their last use
  constexpr int kSumLoad = SUMMARY ? CPOL_DEFAULT : CPOL_NT;
  const int lane = threadIdx.x;
  const ChainPos cp = chain_pos(a);
  const int b = cp.b, mb = cp.mb, t_begin = cp.t_begin, t_end = cp.t_end;
  const int m0 = mb * MB + lane * V;
  const bool lane_ok = m0 < a.M;
  const int n_blocks = (t_end - t_begin + kS - 1) / kS;
  ModeConsts<V, false> mc;
  mc.load(a.consts, m0, lane_ok);
  // the state entering this segment: a buffer load over an empty range (which
  // reads zeros) for the first segment and for summaries.  Not a global load
  // under a branch: that made the compiler restructure the block loop (1.5x
  // slower at B=8, T=4096, width 32768)
  float hr[V], hi[V];
  {
    const bool from_seg = !SUMMARY && a.n_seg > 1;
    const float* base = a.seg_state + (static_cast<int64_t>(b) * a.n_seg + cp.seg) * a.M * 2;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(from_seg ? base : a.consts, from_seg ? a.M * 8u : 0u);
    float h0[2 * V];
    buffer_load_f32<2 * V, CPOL_DEFAULT>(rs, static_cast<uint32_t>(lane_ok ? m0 * 8 : 0), h0);
#pragma unroll
    for (int v = 0; v < V; ++v) {
      hr[v] = h0[2 * v];
      hi[v] = h0[2 * v + 1];
    }
    if constexpr (GW && !SUMMARY) {
      // the caller's initial state, for a single segment (with segments the
      // carry kernel has folded it into the entering state of segment 0)
      const bool from_h0 = a.n_seg == 1 && a.h0_re != nullptr;
      const int64_t hb = static_cast<int64_t>(b) * a.M;
      const __amdgpu_buffer_rsrc_t rr = make_rsrc(from_h0 ? a.h0_re + hb : a.consts, from_h0 ? a.M * 4u : 0u);
      const __amdgpu_buffer_rsrc_t ri = make_rsrc(from_h0 ? a.h0_im + hb : a.consts, from_h0 ? a.M * 4u : 0u);
      float qr[V], qi[V];
      buffer_load_f32<V, CPOL_DEFAULT>(rr, static_cast<uint32_t>(lane_ok ? m0 * 4 : 0), qr);
      buffer_load_f32<V, CPOL_DEFAULT>(ri, static_cast<uint32_t>(lane_ok ? m0 * 4 : 0), qi);
#pragma unroll
      for (int v = 0; v < V; ++v) {
        hr[v] += qr[v];
        hi[v] += qi[v];
      }
    }
  }
  float Pr[V], Pi[V];  // SUMMARY: the product of the segment's transitions
#pragma unroll
  for (int v = 0; v < V; ++v) { Pr[v] = 1.0f; Pi[v] = 0.0f; }
  const int64_t row0 = static_cast<int64_t>(b) * a.T;
  const int64_t mbase = static_cast<int64_t>(mb) * MB;
  const int64_t W = 2 * static_cast<int64_t>(a.M);
  const uint32_t lane_bytes = static_cast<uint32_t>(lane * V * ESZ);
  const uint32_t lane_ld = lane_ok ? lane_bytes : 0u;
  const uint32_t lane_st = lane_ok ? lane_bytes : kDropOffset;
  // bytes of one row of x (2M) and of h (M), and of kS rows (< 2^31: the host
  // limits M to 2^24)
  const uint32_t row_x = static_cast<uint32_t>(W * ESZ), half_x = static_cast<uint32_t>(a.M * ESZ);
  const uint32_t blk_x = kS * row_x, blk_h = kS * half_x;
  // the constants are loop-carried: complete their loads before the loop (else
  // the waits inside it would also cover the prefetch)
  wait_vm_all();

  RawT xr[2][kS], xi[2][kS];
  float ev[2], dv[2];  // lane s < kS: eta, delta of step s of the block
  int kv[2];           // RST: lane s < kS: whether step s keeps its transition
  auto load_block = [&](auto h_tag, int k) {
    constexpr int h = decltype(h_tag)::value;
    const int t0 = t_begin + k * kS;
    const int last = t_end - 1 - t0;
    // the block's rows of x through one buffer resource: row offsets in
    // scalar registers, no per-lane address arithmetic
    if constexpr (GW) {  // the writes: rows of the w_re and w_im planes
      const int64_t off = wave_uniform(((row0 + t0) * a.M + mbase) * ESZ);
      const __amdgpu_buffer_rsrc_t rwr = make_rsrc(static_cast<const char*>(a.w_re) + off, blk_h);
      const __amdgpu_buffer_rsrc_t rwi = make_rsrc(static_cast<const char*>(a.w_im) + off, blk_h);
#pragma unroll
      for (int s = 0; s < kS; ++s) {
        const uint32_t o = static_cast<uint32_t>(s <= last ? s : last) * half_x;
        xr[h][s] = buf_load<RawT, kSumLoad>(rwr, lane_ld, o);
        xi[h][s] = buf_load<RawT, kSumLoad>(rwi, lane_ld, o);
      }
    } else {
      const int64_t off = wave_uniform(((row0 + t0) * W + mbase) * ESZ);
      const __amdgpu_buffer_rsrc_t rx = make_rsrc(static_cast<const char*>(a.x) + off, blk_x);
#pragma unroll
      for (int s = 0; s < kS; ++s) {
        const uint32_t o = static_cast<uint32_t>(s <= last ? s : last) * row_x;
        xr[h][s] = buf_load<RawT, CPOL_NT>(rx, lane_ld, o);
        xi[h][s] = buf_load<RawT, CPOL_NT>(rx, lane_ld, o + half_x);
      }
    }
    const int sl = lane & (kS - 1);
    const int64_t ti = row0 + t0 + (sl <= last ? sl : last);
    ev[h] = a.eta[ti];
    dv[h] = a.delta[ti];
    if constexpr (RST) kv[h] = p1_keep(a, b, t0 + (sl <= last ? sl : last));
  };

  // One block of kS steps in two phases: (A) every step's transition and
  // write, independent of the state, as one straight-line region the
  // compiler can interleave; (B) the recurrence and the stores.  TAIL: the
  // last block, with steps past T (no update, no store).
  auto run_block = [&](auto h_tag, int t0, auto tail_tag) {
    constexpr int h = decltype(h_tag)::value;
    constexpr bool TAIL = decltype(tail_tag)::value;
    float ar[kS][V], ai[kS][V], wr[kS][V], wi[kS][V];
    const float ee = fast_exp(ev[h]);  // lane s: e^eta of step s
    float Es[kS], Ds[kS], Rs[kS];
    p1_block_steps<kS>(ee, dv[h], Es, Ds, Rs);
    if constexpr (GW) {
      float em[kS][V];
      p1_block_transitions<IO, MODE, kS, V>(mc, Es, Ds, Rs, ar, ai, em);
    }
    if constexpr (RST) p1_block_resets<kS, V>(kv[h], ar, ai);
#pragma unroll
    for (int s = 0; s < kS; ++s) {
      float cr[V], ci[V];
      unpack<IO, V>(xr[h][s], cr);
      unpack<IO, V>(xi[h][s], ci);
#pragma unroll
      for (int v = 0; v < V; ++v) {
        if constexpr (GW) {  // the transitions above
          wr[s][v] = cr[v];
          wi[s][v] = ci[v];
        } else {
          const float eta = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(ev[h]), s));
          const StepMode q = p1_step<P1Math<IO, MODE>::HW>(mc.nu[v], mc.ct[v], mc.st[v], mc.g2[v], mc.pl[v],
                                                           mc.rl[v], Es[s], eta, Ds[s], Rs[s]);
          ar[s][v] = q.ar;
          ai[s][v] = q.ai;
          wr[s][v] = q.gain * tanh_fast(cr[v]);
          wi[s][v] = q.gain * tanh_fast(ci[v]);
          if constexpr (kRoundWrite<IO>) round_bf16x2(wr[s][v], wi[s][v]);
        }
      }
    }
    if constexpr (SUMMARY) {
      // the segment's map from a zero state, last step first: with P the
      // product of the transitions after step t, the end state is the sum of
      // P w_t (hr, hi += P w_t, then P <- P a_t); at the end P is the
      // product over the whole segment
#pragma unroll
      for (int s = kS - 1; s >= 0; --s) {
        if (TAIL && t0 + s >= t_end) continue;  // wave-uniform
#pragma unroll
        for (int v = 0; v < V; ++v) {
          hr[v] = fmaf(Pr[v], wr[s][v], fmaf(-Pi[v], wi[s][v], hr[v]));
          hi[v] = fmaf(Pr[v], wi[s][v], fmaf(Pi[v], wr[s][v], hi[v]));
          const float pr = fmaf(ar[s][v], Pr[v], -ai[s][v] * Pi[v]);
          Pi[v] = fmaf(ai[s][v], Pr[v], ar[s][v] * Pi[v]);
          Pr[v] = pr;
        }
      }
      return;
    }
    const int64_t yoff = wave_uniform(((row0 + t0) * W + mbase) * ESZ);
    const int64_t hoff = wave_uniform(((row0 + t0) * a.M + mbase) * ESZ);
    const __amdgpu_buffer_rsrc_t ry = make_rsrc(static_cast<char*>(a.y) + yoff, blk_x);
    const __amdgpu_buffer_rsrc_t rhr = make_rsrc(static_cast<char*>(a.h_re) + hoff, blk_h);
    const __amdgpu_buffer_rsrc_t rhi = make_rsrc(static_cast<char*>(a.h_im) + hoff, blk_h);
#pragma unroll
    for (int s = 0; s < kS; ++s) {
      if (TAIL && t0 + s >= t_end) break;  // wave-uniform
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const float nr = fmaf(ar[s][v], hr[v], fmaf(-ai[s][v], hi[v], wr[s][v]));
        const float ni = fmaf(ai[s][v], hr[v], fmaf(ar[s][v], hi[v], wi[s][v]));
        hr[v] = nr;
        hi[v] = ni;
      }
      if constexpr (CM != kPlanes) {  // y = relu(cat(h_re, h_im))
        float rr[V], ri[V];
#pragma unroll
        for (int v = 0; v < V; ++v) { rr[v] = fmaxf(hr[v], 0.0f); ri[v] = fmaxf(hi[v], 0.0f); }
        const uint32_t yo = static_cast<uint32_t>(s) * row_x;
        buf_store<RawT, CPOL_NT>(pack<IO, V>(rr), ry, lane_st, yo);
        buf_store<RawT, CPOL_NT>(pack<IO, V>(ri), ry, lane_st, yo + half_x);
      }
      if constexpr (CM != kRelu) {  // the states
        const uint32_t ho = static_cast<uint32_t>(s) * half_x;
        buf_store<RawT, CPOL_NT>(pack<IO, V>(hr), rhr, lane_st, ho);
        buf_store<RawT, CPOL_NT>(pack<IO, V>(hi), rhi, lane_st, ho);
      }
    }
    if constexpr (GW && !SUMMARY) {
      // the state after the last step of every 64-step chunk and after T-1
      const int t_last = (TAIL ? t_end : t0 + kS) - 1;
      if ((t_last + 1) % kStateChunk == 0 || t_last == a.T - 1) {  // wave-uniform
        const int64_t n_chunks = (a.T + kStateChunk - 1) / kStateChunk;
        const int64_t off = wave_uniform(((static_cast<int64_t>(b) * n_chunks + t_last / kStateChunk) * a.M + mbase) * 8);
        const __amdgpu_buffer_rsrc_t rc = make_rsrc(reinterpret_cast<char*>(a.chunk_state) + off, MB * 8u);
        float o[2 * V];
#pragma unroll
        for (int v = 0; v < V; ++v) { o[2 * v] = hr[v]; o[2 * v + 1] = hi[v]; }
        buffer_store_f32<2 * V, CPOL_DEFAULT>(rc, lane_ok ? static_cast<uint32_t>(lane * V * 8) : kDropOffset, o);
      }
    }
  };
  // block k uses register buffer k & 1; the loop runs over pairs of blocks so
  // that every buffer index is a compile-time constant (a runtime index into
  // register arrays becomes indexed register access)
  // A summary walks its segment last block first (blk), so that the rows it
  // read last, still in the caches when the replay starts, are the ones the
  // replay reads first.
  auto blk = [&](int k) { return SUMMARY ? n_blocks - 1 - k : k; };
  auto step_block = [&](auto h_tag, int k) {
    constexpr int h = decltype(h_tag)::value;
    load_block(std::integral_constant<int, 1 - h>{}, blk(k + 1 < n_blocks ? k + 1 : k));
    const int t0 = t_begin + blk(k) * kS;
    if (t0 + kS <= t_end) run_block(h_tag, t0, std::false_type{});
    else run_block(h_tag, t0, std::true_type{});
  };
  load_block(std::integral_constant<int, 0>{}, blk(0));
  for (int k = 0; k < n_blocks; k += 2) {
    step_block(std::integral_constant<int, 0>{}, k);
    if (k + 1 < n_blocks) step_block(std::integral_constant<int, 1>{}, k + 1);
  }
  if constexpr (SUMMARY) {
    if (lane_ok) {
#pragma unroll
      for (int v = 0; v < V; ++v)
        *reinterpret_cast<float4*>(a.seg_sum + ((static_cast<int64_t>(b) * a.n_seg + cp.seg) * a.M + m0 + v) * 4) =
            make_float4(Pr[v], Pi[v], hr[v], hi[v]);
    }
  } else if (lane_ok && a.last_re && cp.seg == a.n_seg - 1) {
#pragma unroll
    for (int v = 0; v < V; ++v) {
      a.last_re[static_cast<int64_t>(b) * a.M + m0 + v] = hr[v];
      a.last_im[static_cast<int64_t>(b) * a.M + m0 + v] = hi[v];
    }
  }
}

// ---------------------------------------------------------------------------
// forward over wide chains: one streaming wave and NH helper waves
// ---------------------------------------------------------------------------
// A chain is a batch row and 256 modes (4 per lane), so that every load and
// store moves a 512-byte piece of a row (1 KB for fp32) instead of the
// 128-byte pieces of one mode per lane.  Wave 0 runs the recurrence and the
// stores; waves 1 .. NH load x (kModule) or the writes (kPlanes, kRelu) and
// compute each step's transition and write (the transcendental part of a
// step, SPH = S/NH steps of a block each) into an LDS table one block ahead
// of wave 0, double-buffered, with one workgroup barrier per block.  The
// arithmetic is that of mixer_fwd_kernel in the same chain mode, value for
// value, so both give the same bits.  No time segments: the host takes this
// kernel only with enough chains to fill the GPU.
template <typename IO, int NH, int S, int MODE>
__global__ void __launch_bounds__(64 * (NH + 1))
mixer_fwd_wide_kernel(Args a) {
  constexpr int V = 4;
  constexpr int MB = 64 * V;
  constexpr int ESZ = sizeof(IO);
  constexpr int SPH = S / NH;  // steps of a block per helper wave
  static_assert(S % NH == 0 && SPH <= 64 && kStateChunk % S == 0, "whole steps per helper, blocks tile the chunks");
  constexpr int CM = MODE & 3;             // the chain mode without kReset
  constexpr bool RST = (MODE & kReset) != 0;
  constexpr bool GW = CM != kModule;       // the writes are given
  static_assert(GW || !RST, "resets in the P1 scan only");
  constexpr bool PACKW = sizeof(IO) == 2;  // bf16 writes: one dword (re | im << 16) per mode
  static_assert(GW || PACKW == kRoundWrite<IO>, "the module's bf16 writes are rounded to bf16");
  constexpr int NPL = PACKW ? 3 : 4;       // table planes per step: ar, ai, then w or wr, wi
  using RawT = typename Raw<IO, V>::T;
  __shared__ float4 tab[2][S][NPL][64];  // [buffer][step][plane][lane]: the lane's 4 modes

  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));  // wave-uniform
  // the streaming wave is the block pipeline's critical path: it issues ahead
  // of the helpers that share its SIMD (P1 forward at B=8, T=4096, M=16384,
  // two boxes: 0.741-0.743 -> 0.721-0.722 ms and 0.757-0.759 -> 0.734-0.736
  // ms; the helpers first instead: 0.79 ms; module forward about 1 % faster)
  if (wave == 0) __builtin_amdgcn_s_setprio(3);
  const int lane = threadIdx.x & 63;
  const int idx = xcd_swizzle(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x));
  const int b = idx / a.n_mb, mb = idx - b * a.n_mb;
  const int m0 = mb * MB + lane * V;
  const bool lane_ok = m0 < a.M;  // the host requires M % 4 == 0: a lane's modes are all in or all out
  const int T = a.T;
  const int n_blocks = (T + S - 1) / S;
  const int64_t row0 = static_cast<int64_t>(b) * T;
  const int64_t mbase = static_cast<int64_t>(mb) * MB;
  const int64_t W = 2 * static_cast<int64_t>(a.M);
  const uint32_t lane_bytes = static_cast<uint32_t>(lane * V * ESZ);
  const uint32_t lane_ld = lane_ok ? lane_bytes : 0u;
  const uint32_t lane_st = lane_ok ? lane_bytes : kDropOffset;
  // bytes of one row of x / y (2M) and of h / w (M) (< 2^31: the host limits M to 2^24)
  const uint32_t row_x = static_cast<uint32_t>(W * ESZ), half_x = static_cast<uint32_t>(a.M * ESZ);

  // helpers: the per-mode constants and, double-buffered in registers, the
  // rows of x or of the writes and (lane j < SPH) eta, delta (and whether the
  // step keeps its transition) of their steps of a block
  const int hw = wave > 0 ? wave - 1 : 0;
  ModeConsts<V, false> mc;
  mc.load(a.consts, m0, lane_ok);
  RawT xr[2][SPH], xi[2][SPH];
  float ev[2], dv[2];
  int kv[2];
  // wave 0: the state, from the caller's initial state (the P1 scan) or zero
  float hr[V], hi[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const bool h0 = GW && wave == 0 && lane_ok && a.h0_re != nullptr;
    hr[v] = h0 ? a.h0_re[static_cast<int64_t>(b) * a.M + m0 + v] : 0.0f;
    hi[v] = h0 ? a.h0_im[static_cast<int64_t>(b) * a.M + m0 + v] : 0.0f;
  }
  wait_vm_all();  // the loop-carried constants and state, before the first prefetch

  // rows past T re-read row T-1 (no loads under a branch)
  auto load_block = [&](auto h_tag, int k) __attribute__((always_inline)) {
    constexpr int h = decltype(h_tag)::value;
    const int t0 = k * S + hw * SPH;
    const int tb = min(t0, T - 1);
    if constexpr (GW) {
      const int64_t off = wave_uniform(((row0 + tb) * a.M + mbase) * ESZ);
      const __amdgpu_buffer_rsrc_t rwr = make_rsrc(static_cast<const char*>(a.w_re) + off, SPH * half_x);
      const __amdgpu_buffer_rsrc_t rwi = make_rsrc(static_cast<const char*>(a.w_im) + off, SPH * half_x);
#pragma unroll
      for (int j = 0; j < SPH; ++j) {
        const uint32_t o = static_cast<uint32_t>(min(t0 + j, T - 1) - tb) * half_x;
        xr[h][j] = buf_load<RawT, CPOL_NT>(rwr, lane_ld, o);
        xi[h][j] = buf_load<RawT, CPOL_NT>(rwi, lane_ld, o);
      }
    } else {
      const int64_t off = wave_uniform(((row0 + tb) * W + mbase) * ESZ);
      const __amdgpu_buffer_rsrc_t rx = make_rsrc(static_cast<const char*>(a.x) + off, SPH * row_x);
#pragma unroll
      for (int j = 0; j < SPH; ++j) {
        const uint32_t o = static_cast<uint32_t>(min(t0 + j, T - 1) - tb) * row_x;
        xr[h][j] = buf_load<RawT, CPOL_NT>(rx, lane_ld, o);
        xi[h][j] = buf_load<RawT, CPOL_NT>(rx, lane_ld, o + half_x);
      }
    }
    const int tl = min(t0 + lane % SPH, T - 1);
    ev[h] = a.eta[row0 + tl];
    dv[h] = a.delta[row0 + tl];
    if constexpr (RST) kv[h] = p1_keep(a, b, tl);
  };
  // a helper's steps of one block into table buffer kb
  auto compute_block = [&](auto h_tag, int kb) __attribute__((always_inline)) {
    constexpr int h = decltype(h_tag)::value;
    const float ee = fast_exp(ev[h]);  // lane j: e^eta of step j
    float Es[SPH], Ds[SPH], Rs[SPH];
    p1_block_steps<SPH>(ee, dv[h], Es, Ds, Rs);
#pragma unroll
    for (int j = 0; j < SPH; ++j) {
      float ar[V], ai[V];
      float4 w0, w1;  // the table's write plane(s)
      if constexpr (GW) {
        // the transition of p1_block_transitions, a := 0 at a reset step
        const bool keep = !RST || __builtin_amdgcn_readlane(kv[h], j) != 0;  // wave-uniform
        float a1r[1][V], a1i[1][V], em[1][V];
        const float E1[1] = {Es[j]}, D1[1] = {Ds[j]}, R1[1] = {Rs[j]};
        p1_block_transitions<IO, MODE, 1, V>(mc, E1, D1, R1, a1r, a1i, em);
#pragma unroll
        for (int v = 0; v < V; ++v) {
          ar[v] = keep ? a1r[0][v] : 0.0f;
          ai[v] = keep ? a1i[0][v] : 0.0f;
        }
        if constexpr (PACKW) {  // the raw bf16 writes, re in the low half of each dword
          const uint32_t* r = reinterpret_cast<const uint32_t*>(&xr[h][j]);
          const uint32_t* i = reinterpret_cast<const uint32_t*>(&xi[h][j]);
          w0.x = __uint_as_float((r[0] & 0xffffu) | (i[0] << 16));
          w0.y = __uint_as_float((r[0] >> 16) | (i[0] & 0xffff0000u));
          w0.z = __uint_as_float((r[1] & 0xffffu) | (i[1] << 16));
          w0.w = __uint_as_float((r[1] >> 16) | (i[1] & 0xffff0000u));
        } else {
          float wr[V], wi[V];
          unpack<IO, V>(xr[h][j], wr);
          unpack<IO, V>(xi[h][j], wi);
          w0 = make_float4(wr[0], wr[1], wr[2], wr[3]);
          w1 = make_float4(wi[0], wi[1], wi[2], wi[3]);
        }
      } else {
        float cr[V], ci[V], wr[V], wi[V];
        unpack<IO, V>(xr[h][j], cr);
        unpack<IO, V>(xi[h][j], ci);
        const float eta = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(ev[h]), j));
#pragma unroll
        for (int v = 0; v < V; ++v) {
          const StepMode q = p1_step<P1Math<IO, MODE>::HW>(mc.nu[v], mc.ct[v], mc.st[v], mc.g2[v], mc.pl[v],
                                                           mc.rl[v], Es[j], eta, Ds[j], Rs[j]);
          ar[v] = q.ar;
          ai[v] = q.ai;
          wr[v] = q.gain * tanh_fast(cr[v]);
          wi[v] = q.gain * tanh_fast(ci[v]);
        }
        if constexpr (PACKW) {  // rounded to bf16, as round_bf16x2
          w0.x = __uint_as_float(pack_bf16x2(wr[0], wi[0]));
          w0.y = __uint_as_float(pack_bf16x2(wr[1], wi[1]));
          w0.z = __uint_as_float(pack_bf16x2(wr[2], wi[2]));
          w0.w = __uint_as_float(pack_bf16x2(wr[3], wi[3]));
        } else {
          w0 = make_float4(wr[0], wr[1], wr[2], wr[3]);
          w1 = make_float4(wi[0], wi[1], wi[2], wi[3]);
        }
      }
      const int s = hw * SPH + j;
      tab[kb][s][0][lane] = make_float4(ar[0], ar[1], ar[2], ar[3]);
      tab[kb][s][1][lane] = make_float4(ai[0], ai[1], ai[2], ai[3]);
      tab[kb][s][2][lane] = w0;
      if constexpr (!PACKW) tab[kb][s][NPL - 1][lane] = w1;
    }
  };
  // wave 0: block k from table buffer k & 1
  auto stream_block = [&](int k) __attribute__((always_inline)) {
    const int t0 = k * S, kb = k & 1;
    const int64_t yoff = wave_uniform(((row0 + t0) * W + mbase) * ESZ);
    const int64_t hoff = wave_uniform(((row0 + t0) * a.M + mbase) * ESZ);
    const __amdgpu_buffer_rsrc_t ry = make_rsrc(static_cast<char*>(a.y) + yoff, CM != kPlanes ? S * row_x : 0u);
    const __amdgpu_buffer_rsrc_t rhr = make_rsrc(static_cast<char*>(a.h_re) + hoff, CM != kRelu ? S * half_x : 0u);
    const __amdgpu_buffer_rsrc_t rhi = make_rsrc(static_cast<char*>(a.h_im) + hoff, CM != kRelu ? S * half_x : 0u);
#pragma unroll
    for (int s = 0; s < S; ++s) {
      if (t0 + s >= T) break;  // wave-uniform
      const float4 A = tab[kb][s][0][lane], Bv = tab[kb][s][1][lane], C = tab[kb][s][2][lane];
      const float ar[V] = {A.x, A.y, A.z, A.w}, ai[V] = {Bv.x, Bv.y, Bv.z, Bv.w};
      float wr[V], wi[V];
      if constexpr (PACKW) {
        const float c4[V] = {C.x, C.y, C.z, C.w};
#pragma unroll
        for (int v = 0; v < V; ++v) {
          const uint32_t u = __float_as_uint(c4[v]);
          wr[v] = __uint_as_float(u << 16);
          wi[v] = __uint_as_float(u & 0xffff0000u);
        }
      } else {
        const float4 D = tab[kb][s][NPL - 1][lane];
        wr[0] = C.x; wr[1] = C.y; wr[2] = C.z; wr[3] = C.w;
        wi[0] = D.x; wi[1] = D.y; wi[2] = D.z; wi[3] = D.w;
      }
      float rr[V], ri[V];
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const float nr = fmaf(ar[v], hr[v], fmaf(-ai[v], hi[v], wr[v]));
        const float ni = fmaf(ai[v], hr[v], fmaf(ar[v], hi[v], wi[v]));
        hr[v] = nr;
        hi[v] = ni;
        rr[v] = fmaxf(nr, 0.0f);
        ri[v] = fmaxf(ni, 0.0f);
      }
      if constexpr (CM != kPlanes) {  // y = relu(cat(h_re, h_im))
        const uint32_t yo = static_cast<uint32_t>(s) * row_x;
        buf_store<RawT, CPOL_NT>(pack<IO, V>(rr), ry, lane_st, yo);
        buf_store<RawT, CPOL_NT>(pack<IO, V>(ri), ry, lane_st, yo + half_x);
      }
      if constexpr (CM != kRelu) {  // the states
        const uint32_t ho = static_cast<uint32_t>(s) * half_x;
        buf_store<RawT, CPOL_NT>(pack<IO, V>(hr), rhr, lane_st, ho);
        buf_store<RawT, CPOL_NT>(pack<IO, V>(hi), rhi, lane_st, ho);
      }
    }
    if constexpr (GW) {
      // the state after the last step of every 64-step chunk and after T-1
      const int t_last = min(t0 + S, T) - 1;
      if ((t_last + 1) % kStateChunk == 0 || t_last == T - 1) {  // wave-uniform
        const int64_t n_chunks = (T + kStateChunk - 1) / kStateChunk;
        const int64_t off = wave_uniform(((static_cast<int64_t>(b) * n_chunks + t_last / kStateChunk) * a.M + mbase) * 8);
        const __amdgpu_buffer_rsrc_t rc = make_rsrc(reinterpret_cast<char*>(a.chunk_state) + off, MB * 8u);
        const float o0[4] = {hr[0], hi[0], hr[1], hi[1]}, o1[4] = {hr[2], hi[2], hr[3], hi[3]};
        const uint32_t co = static_cast<uint32_t>(lane * V * 8);
        buffer_store_f32<4, CPOL_DEFAULT>(rc, lane_ok ? co : kDropOffset, o0);
        buffer_store_f32<4, CPOL_DEFAULT>(rc, lane_ok ? co + 16u : kDropOffset, o1);
      }
    }
  };
  // iteration k: wave 0 streams block k; the helpers prefetch block k + 2
  // into the registers block k used and build block k + 1's table
  auto iteration = [&](auto h_tag, int k) __attribute__((always_inline)) {
    constexpr int h = decltype(h_tag)::value;  // k & 1
    if (wave == 0) {
      stream_block(k);
    } else if (k + 1 < n_blocks) {
      load_block(h_tag, min(k + 2, n_blocks - 1));
      compute_block(std::integral_constant<int, 1 - h>{}, 1 - h);
    }
    __syncthreads();
  };
  if (wave > 0) {
    load_block(std::integral_constant<int, 0>{}, 0);
    load_block(std::integral_constant<int, 1>{}, min(1, n_blocks - 1));
    compute_block(std::integral_constant<int, 0>{}, 0);
  }
  __syncthreads();
  for (int k = 0; k < n_blocks; k += 2) {
    iteration(std::integral_constant<int, 0>{}, k);
    if (k + 1 < n_blocks) iteration(std::integral_constant<int, 1>{}, k + 1);
  }
  if (wave == 0 && lane_ok && a.last_re) {
#pragma unroll
    for (int v = 0; v < V; ++v) {
      a.last_re[static_cast<int64_t>(b) * a.M + m0 + v] = hr[v];
      a.last_im[static_cast<int64_t>(b) * a.M + m0 + v] = hi[v];
    }
  }
}

// ---------------------------------------------------------------------------
// backward scan: one chain per workgroup of two waves, reverse time
// ---------------------------------------------------------------------------
// Per step t and mode, with lambda the adjoint of h_t and h' = h_{t-1}:
//   dx          = lambda * gain * (1 - tanh^2 x)              (the write)
//   g           = (lambda_re tanh x_re + lambda_im tanh x_im) * gain
//   dA          = lambda * conj(h')  -> (gar, gai)
//   dphi        = -gar a_im + gai a_re
//   radial      = log(rho) (gar a_re + gai a_im) - log(rho) rho delta dphi
//   wterm       = z rho^2 / (1 - rho^2),  z = nu e^eta   (d log ratio / d eta)
//   d eta_t    += radial + g (wterm + (1 - sig) wrr / log16)
//   d delta_t  += dphi (1 - rho) + g (1 - sig) wpr 2/pi
//   d nu_log   += radial + g (wterm - kappa),  kappa = nu e^{-2nu} / (1 - e^{-2nu})
//   d theta_log+= theta dphi
//   d wlg += g, d wpr += g (1 - sig) delta 2/pi, d wrr += g (1 - sig) eta / log16
// (the P1 chain rule of sparc-kernal/backward/scan.py:593-644 and the write
// gradients of sparc-kernal/backward/control.py:10-89).
// two waves per SIMD; one for the P1 scan's 16-step blocks (about 256 VGPRs)
//
// kCoop (the module, one launch over all T, every chain resident at once):
// the controls' backward runs inside.  d eta_t and d delta_t are sums over
// all mode blocks of a batch row, known only once every chain of the row has
// passed step t; dx_t needs them (dx += dp_phase u_phase + dp_radial
// u_radial, dp the projections' gradients from d eta, d delta), and so do
// the direction gradients (sum_t dp_t x_t).  So each chain stores its wave
// sums of each block (its record, agent-scope stores, no atomics).  Each
// block has one owner, the chain whose mode block is the block index mod
// n_mb: from two blocks later it polls the row's records at its block ends
// and, once none holds the empty marker they start as, sums them in a fixed
// order (the result does not depend on timing), turns them into dp and
// stores them.  A chain keeps each block's dx (rounded to the I/O type) and
// x in an LDS ring and completes the block kCoopLag blocks later, once dp
// differs from the marker (reducing it first if it owns the block and has
// not yet).  Every step of this exchange waits only on memory
// operations issued a block earlier, so the blocks' compute hides it.  A wait
// depends only on blocks every chain passes before it waits itself, so it
// ends once all chains of the row are resident (the host launches this form
// only when the grid fits the GPU at the kernel's occupancy); it is bounded
// anyway (coop_spin polls), after which the error word is set and the
// block's gradients are NaN.  Replaces the controls-backward launches and
// the dx round trip between them (sparc-kernal/backward/control.py:10-89 for
// the controls' chain rule).
template <typename IO, int V, int kS, bool SUMMARY, int MODE>
__global__ void __launch_bounds__(64, (MODE & 3) == kPlanes && kS >= 16 ? 1 : 2)
mixer_bwd_kernel(Args a) {
  using RawT = typename Raw<IO, V>::T;
  constexpr int ESZ = sizeof(IO);
  constexpr int MB = 64 * V;
  constexpr int CM = MODE & 3;             // the chain mode without kReset
  constexpr bool RST = (MODE & kReset) != 0;
  constexpr bool COOP = (MODE & kCoop) != 0;
  constexpr bool GW = CM == kPlanes;  // the writes are given: dw out, no relu mask
  static_assert(CM != kRelu, "the backward of the relu output recomputes states (scan.hip)");
  static_assert(GW || !RST, "resets in the P1 scan only");
  static_assert(!COOP || (CM == kModule && V == 1 && !SUMMARY), "one-launch form: the module, one mode per lane");
  constexpr int kSumLoad = SUMMARY ? CPOL_DEFAULT : CPOL_NT;  // as in mixer_fwd_kernel
  __shared__ float4 tok[64];  // the block's per-step values (run_block)
  const int lane = threadIdx.x;
  const ChainPos cp = chain_pos(a);
  const int b = cp.b, mb = cp.mb, t_begin = cp.t_begin, t_end = cp.t_end;
  const int m0 = mb * MB + lane * V;
  const bool lane_ok = m0 < a.M;
  const int n_blocks = (t_end - t_begin + kS - 1) / kS;
  const int64_t R = static_cast<int64_t>(a.B) * a.T;
  const int64_t row0 = static_cast<int64_t>(b) * a.T;
  // per-token partials: columns b*T + t of [2][n_mb][B*T], or, in time
  // pieces, columns b*t_seg + t - t_begin of piece s's [2][n_mb][B*t_seg]
  const int64_t Rp = a.piped ? static_cast<int64_t>(a.B) * a.t_seg : R;
  const int64_t tok0 =
      a.piped ? static_cast<int64_t>(cp.seg) * 2 * a.n_mb * Rp + static_cast<int64_t>(b) * a.t_seg - t_begin : row0;
  const int64_t mbase = static_cast<int64_t>(mb) * MB;
  const int64_t W = 2 * static_cast<int64_t>(a.M);
  const uint32_t lane_bytes = static_cast<uint32_t>(lane * V * ESZ);
  const uint32_t lane_ld = lane_ok ? lane_bytes : 0u;
  const uint32_t lane_st = lane_ok ? lane_bytes : kDropOffset;
  // bytes of one row of x / dy / dx (2M) and of h (M), and of kS rows (the host
  // limits M to 2^24, so these fit in 32 bits)
  const uint32_t row_x = static_cast<uint32_t>(W * ESZ), half_x = static_cast<uint32_t>(a.M * ESZ);
  const uint32_t blk_x = kS * row_x, blk_h = kS * half_x;

  ModeConsts<V, true> mc;
  mc.load(a.consts, m0, lane_ok);
  // kCoop: the directions at this lane's channels (phase re, radial re, phase
  // im, radial im), the direction-gradient sums in the same order, the ring
  // of the blocks waiting for their controls gradient (block k in slot
  // k % L), the next such gradient to use (loaded one block ahead) and the
  // block this chain is to reduce and has not yet (-1: none)
  constexpr int L = COOP ? kCoopLag<IO> : 1;
  __shared__ typename CoopRing<IO>::T cring[L][COOP ? kS : 1][64];
  float cu[4], ad[4], dpn[COOP ? 2 * kS : 1];
  int pend = -1;
  if constexpr (COOP) {
    const int mm = lane_ok ? m0 : 0;
    cu[0] = lane_ok ? a.pdir[mm] : 0.0f;
    cu[1] = lane_ok ? a.rdir[mm] : 0.0f;
    cu[2] = lane_ok ? a.pdir[a.M + mm] : 0.0f;
    cu[3] = lane_ok ? a.rdir[a.M + mm] : 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) ad[i] = 0.0f;
#pragma unroll
    for (int i = 0; i < 2 * kS; ++i) dpn[i] = __uint_as_float(kCoopEmpty);
  }
  float Xr[V], Xi[V];    // conj(a_{t+1}) lambda_{t+1}
  float hcr[V], hci[V];  // h at the last step of the next block to process
  float acc[5][V];       // nu_log, theta_log, wlg, wpr, wrr
  float Pr[V], Pi[V];    // SUMMARY: the product of the segment's conj(a)
#pragma unroll
  for (int v = 0; v < V; ++v) {
    // the adjoint entering this segment from the right (summaries start at zero)
    const int64_t i0 = static_cast<int64_t>(b) * a.M + (lane_ok ? m0 + v : 0);
    if (SUMMARY) {
      Xr[v] = 0.0f;
      Xi[v] = 0.0f;
    } else if (a.n_seg > 1 && !(a.piped && cp.seg == a.n_seg - 1)) {
      const float2 x0 = *reinterpret_cast<const float2*>(
          a.seg_state + ((static_cast<int64_t>(b) * a.n_seg + cp.seg) * a.M + (lane_ok ? m0 + v : 0)) * 2);
      Xr[v] = x0.x;
      Xi[v] = x0.y;
    } else {
      Xr[v] = a.dlast_re ? a.dlast_re[i0] : 0.0f;
      Xi[v] = a.dlast_im ? a.dlast_im[i0] : 0.0f;
    }
    Pr[v] = 1.0f;
    Pi[v] = 0.0f;
#pragma unroll
    for (int p = 0; p < 5; ++p) acc[p][v] = 0.0f;
  }
  if constexpr (!GW) {  // h at the segment's last step: its relu mask
    const int64_t ho = wave_uniform(((row0 + t_end - 1) * a.M + mbase) * ESZ);
    unpack<IO, V>(ldb<RawT>(a.h_re, ho, lane_ld), hcr);
    unpack<IO, V>(ldb<RawT>(a.h_im, ho, lane_ld), hci);
  }
  // GW: the state before step 0 (the caller's initial state, else zero), for
  // the transition gradient of step 0; a buffer load over an empty range
  // reads the zeros
  float h0r[V], h0i[V];
  if constexpr (GW && !SUMMARY) {
    const bool use = t_begin == 0 && a.h0_re != nullptr;
    const int64_t hb = static_cast<int64_t>(b) * a.M;
    const __amdgpu_buffer_rsrc_t rr = make_rsrc(use ? a.h0_re + hb : a.consts, use ? a.M * 4u : 0u);
    const __amdgpu_buffer_rsrc_t ri = make_rsrc(use ? a.h0_im + hb : a.consts, use ? a.M * 4u : 0u);
    buffer_load_f32<V, CPOL_DEFAULT>(rr, static_cast<uint32_t>(lane_ok ? m0 * 4 : 0), h0r);
    buffer_load_f32<V, CPOL_DEFAULT>(ri, static_cast<uint32_t>(lane_ok ? m0 * 4 : 0), h0i);
  } else {
#pragma unroll
    for (int v = 0; v < V; ++v) { h0r[v] = 0.0f; h0i[v] = 0.0f; }
  }
  wait_vm_all();  // the loop-carried values above, before the first prefetch

  RawT dr[2][kS], di[2][kS], xr[2][kS], xi[2][kS], pr[2][kS], pi[2][kS];
  float ev[2], dv[2];
  int kv[2];  // RST: lane s < kS: whether step s keeps its transition
  // block k: steps t0 .. t0+kS-1; the previous states are rows t-1 (row 0
  // for t = 0, zeroed in the step)
  auto load_block = [&](auto h_tag, int k) {
    constexpr int h = decltype(h_tag)::value;
    const int t0 = t_begin + k * kS;
    const int last = t_end - 1 - t0;
    // buffer resources over the block's rows (row offsets in scalar
    // registers); the previous states start at row t0-1 (row 0 when t0 = 0)
    const int hb = t0 > 0 ? t0 - 1 : 0;
    const int64_t xoff = wave_uniform(((row0 + t0) * W + mbase) * ESZ);
    const int64_t woff = wave_uniform(((row0 + t0) * a.M + mbase) * ESZ);
    const int64_t poff = wave_uniform(((row0 + hb) * a.M + mbase) * ESZ);
    // module: dy [B,T,2M] and x; GW: the dy_re and dy_im planes [B,T,M]
    const __amdgpu_buffer_rsrc_t rdy = GW ? make_rsrc(static_cast<const char*>(a.dy) + woff, blk_h)
                                          : make_rsrc(static_cast<const char*>(a.dy) + xoff, blk_x);
    const __amdgpu_buffer_rsrc_t rdi = GW ? make_rsrc(static_cast<const char*>(a.dy_im) + woff, blk_h) : rdy;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(static_cast<const char*>(a.x) + xoff, blk_x);
    const __amdgpu_buffer_rsrc_t rpr = make_rsrc(static_cast<const char*>(a.h_re) + poff, blk_h);
    const __amdgpu_buffer_rsrc_t rpi = make_rsrc(static_cast<const char*>(a.h_im) + poff, blk_h);
#pragma unroll
    for (int s = 0; s < kS; ++s) {
      const int sc = s <= last ? s : last;
      if constexpr (GW) {
        const uint32_t o = static_cast<uint32_t>(sc) * half_x;
        dr[h][s] = buf_load<RawT, kSumLoad>(rdy, lane_ld, o);
        di[h][s] = buf_load<RawT, kSumLoad>(rdi, lane_ld, o);
      } else {
        const uint32_t o = static_cast<uint32_t>(sc) * row_x;
        dr[h][s] = buf_load<RawT, kSumLoad>(rdy, lane_ld, o);
        di[h][s] = buf_load<RawT, kSumLoad>(rdy, lane_ld, o + half_x);
        if constexpr (!SUMMARY) {  // summaries need no write path
          xr[h][s] = buf_load<RawT, CPOL_NT>(rx, lane_ld, o);
          xi[h][s] = buf_load<RawT, CPOL_NT>(rx, lane_ld, o + half_x);
        }
      }
      if constexpr (!(GW && SUMMARY)) {  // GW summaries need no states (no relu mask)
        // row t-1 (t >= 1), else row 0, relative to hb
        const int rel = t0 > 0 ? sc : (sc > 0 ? sc - 1 : 0);
        const uint32_t q = static_cast<uint32_t>(rel) * half_x;
        pr[h][s] = buf_load<RawT, CPOL_NT>(rpr, lane_ld, q);
        pi[h][s] = buf_load<RawT, CPOL_NT>(rpi, lane_ld, q);
      }
    }
    const int sl = lane & (kS - 1);
    const int64_t ti = row0 + t0 + (sl <= last ? sl : last);
    ev[h] = a.eta[ti];
    dv[h] = a.delta[ti];
    if constexpr (RST) kv[h] = p1_keep(a, b, t0 + (sl <= last ? sl : last));
  };

  // kCoop helpers.  Records, gradients and counts travel between chains
  // (possibly on different XCDs) through agent-scope (sc1) accesses.
  const int nblk = COOP ? a.coop_nblk : 1;
  const int64_t slot0 = static_cast<int64_t>(b) * nblk;  // this batch row's first block
  constexpr int NV = 2 * kS;                             // per-token values of a block
  constexpr int KV = NV >= 16 ? NV / 16 : 1, GV = 64 * KV / NV;
  // this chain's record of block kb: the leaders' wave sums (value i: d eta
  // of step i/2 for even i, d delta for odd i)
  auto coop_store_record = [&](int kb, const float (&sums)[NV]) __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t rp =
        make_rsrc(a.coop_part + wave_uniform(((slot0 + kb) * a.n_mb + mb) * NV), static_cast<uint32_t>(NV * 4));
#pragma unroll
    for (int k = 0; k < KV; ++k) {
      const float v[1] = {sums[k]};
      buffer_store_f32<1, CPOL_SC1>(rp, lane % GV == 0 ? static_cast<uint32_t>((lane / GV * KV + k) * 4) : kDropOffset,
                                    v);
    }
  };
  // block kc's controls gradient, every lane the same values
  auto coop_load_grad = [&](int kc, float (&v)[NV]) __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.coop_sum + wave_uniform((slot0 + kc) * NV), static_cast<uint32_t>(NV * 4));
#pragma unroll
    for (int j = 0; j < NV / 4; ++j) {
      float t[4];
      buffer_load_f32<4, CPOL_SC1>(rs, static_cast<uint32_t>(16 * j), t);
#pragma unroll
      for (int q = 0; q < 4; ++q) v[4 * j + q] = t[q];
    }
  };
  auto coop_final = [&](const float (&v)[NV]) -> bool {
    bool ok = true;
#pragma unroll
    for (int i = 0; i < NV; ++i) ok = ok && __float_as_uint(v[i]) != kCoopEmpty;
    return __builtin_amdgcn_readfirstlane(static_cast<int>(ok)) != 0;
  };
  // The reduction of block kr by its chain (mode block kr % n_mb of the
  // row): the row's records, once none is kCoopEmpty (else false, or with
  // `wait` loads again, at most coop_spin polls: then the error word), summed
  // in a fixed order (lane l the records l, l + 64, ..., then the wave's
  // sums), turned into the projections' gradients as the controls' backward
  // does (dp_radial = d eta log16 (1 - (eta/log16)^2), dp_phase = d delta
  // pi/2 (1 - (2 delta/pi)^2)) and stored for the row's chains and per token.
  auto coop_reduce = [&](int kr, bool wait) -> bool {
    float r[NV];
    const __amdgpu_buffer_rsrc_t rr =
        make_rsrc(a.coop_part + wave_uniform((slot0 + kr) * a.n_mb * NV), static_cast<uint32_t>(a.n_mb * NV * 4));
    for (uint32_t it = 0;; ++it) {
      bool full = true;
#pragma unroll
      for (int i = 0; i < NV; ++i) r[i] = 0.0f;
      for (int c = lane; c < a.n_mb; c += 64) {
#pragma unroll
        for (int j = 0; j < NV / 4; ++j) {
          float t[4];
          buffer_load_f32<4, CPOL_SC1>(rr, static_cast<uint32_t>((c * NV + 4 * j) * 4), t);
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            full = full && __float_as_uint(t[q]) != kCoopEmpty;
            r[4 * j + q] += t[q];
          }
        }
      }
      if (__builtin_amdgcn_ballot_w64(!full) == 0) break;  // every record complete
      if (!wait) return false;
      const bool failed = it >= a.coop_spin ||
                          ((it & 255u) == 255u && __builtin_amdgcn_readfirstlane(load_agent(a.coop_error)) != 0u);
      if (failed) {
        if (lane == 0) store_agent(a.coop_error, 1u);
#pragma unroll
        for (int i = 0; i < NV; ++i) r[i] = __builtin_nanf("");
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    wave_sums_to_leaders<NV>(r);
    const int t0r = t_begin + kr * kS;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.coop_sum + wave_uniform((slot0 + kr) * NV), static_cast<uint32_t>(NV * 4));
    const bool lead = lane % GV == 0;
#pragma unroll
    for (int k = 0; k < KV; ++k) {
      const int i = lane / GV * KV + k, t = t0r + (i >> 1);
      const bool live = t < t_end;
      const float ee = (live ? a.eta[row0 + t] : 0.0f) * kInvLog16;
      const float dd = (live ? a.delta[row0 + t] : 0.0f) * kTwoOverPi;
      const float dp = (i & 1) ? r[k] * kHalfPi * fmaf(-dd, dd, 1.0f) : r[k] * kLog16 * fmaf(-ee, ee, 1.0f);
      const float v[1] = {dp};
      buffer_store_f32<1, CPOL_SC1>(rs, lead ? static_cast<uint32_t>(i * 4) : kDropOffset, v);
      if (lead && live) a.coop_dtok[((i & 1) ? 0 : R) + row0 + t] = dp;  // [0] phase, [1] radial
    }
    return true;
  };
  // v holds block kc's gradient as loaded earlier; until it is final, load
  // it again (at most coop_spin polls: then the error word, and NaN).  Its
  // own chain reduces it first if it has not yet.
  auto coop_await = [&](int kc, float (&v)[NV]) __attribute__((always_inline)) {
    if (coop_final(v)) return;
    if (kc % a.n_mb == mb) {  // this chain's block: reduce it now unless it has
      coop_load_grad(kc, v);
      if (!coop_final(v)) {
        (void)coop_reduce(kc, true);
        wait_stores_complete();
      }
      if (pend == kc) pend = -1;
      coop_load_grad(kc, v);
      if (coop_final(v)) return;
    }
    for (uint32_t it = 0; it < a.coop_spin; ++it) {
      if ((it & 255u) == 255u && __builtin_amdgcn_readfirstlane(load_agent(a.coop_error)) != 0u) break;
      __builtin_amdgcn_s_sleep(2);
      coop_load_grad(kc, v);
      if (coop_final(v)) return;
    }
    if (lane == 0) store_agent(a.coop_error, 1u);
#pragma unroll
    for (int i = 0; i < NV; ++i) v[i] = __builtin_nanf("");
  };
  // Block kc from its ring slot with its controls gradient dp: dx += dp_phase
  // u_phase + dp_radial u_radial per channel (the controls' backward's order
  // of operations), the direction sums dp x, the dx stores.
  auto coop_finish = [&](int kc, const float (&dp)[NV]) __attribute__((always_inline)) {
    const int sl = kc % L;
    const int t0c = t_begin + kc * kS;
    const int64_t xoff = wave_uniform(((row0 + t0c) * W + mbase) * ESZ);
    const __amdgpu_buffer_rsrc_t rdx = make_rsrc(static_cast<char*>(a.dx) + xoff, blk_x);
#pragma unroll
    for (int s = 0; s < kS; ++s) {
      if (t0c + s >= t_end) break;  // wave-uniform: the block holding T-1
      float dr, di, xr1, xi1;
      CoopRing<IO>::get(cring[sl][s][lane], dr, di, xr1, xi1);
      const float p1 = dp[2 * s], p0 = dp[2 * s + 1];
      const float gr[1] = {fmaf(p0, cu[0], fmaf(p1, cu[1], dr))};
      const float gi[1] = {fmaf(p0, cu[2], fmaf(p1, cu[3], di))};
      ad[0] = fmaf(p0, xr1, ad[0]);
      ad[1] = fmaf(p1, xr1, ad[1]);
      ad[2] = fmaf(p0, xi1, ad[2]);
      ad[3] = fmaf(p1, xi1, ad[3]);
      const uint32_t o = static_cast<uint32_t>(s) * row_x;
      buf_store<typename Raw<IO, 1>::T, CPOL_NT>(pack<IO, 1>(gr), rdx, lane_st, o);
      buf_store<typename Raw<IO, 1>::T, CPOL_NT>(pack<IO, 1>(gi), rdx, lane_st, o + half_x);
    }
  };

  // One block of kS steps: (A) every step's transition (independent of the
  // adjoint), then (B) one pass over the steps in reverse: the adjoint
  // lambda = dy (relu-masked in the module) + X, the write's gradient,
  // X = conj(a) lambda (carried to the step before), and the transition
  // gradients from Z = X conj(h'): for dA = lambda conj(h'), conj(a) dA = Z,
  // so Re Z = gar a_re + gai a_im and Im Z = dphi, and radial = -log(rho)
  // (rho delta Im Z - Re Z) = E nu (rho delta Im Z - Re Z) with the factor E
  // of the step taken out of the per-mode products; then (C) the stores and
  // the wave sums of the per-token gradients.  Straight-line code the
  // compiler can interleave across steps.
  // TAIL: the block holding T-1 when T is not a multiple of kS.  The relu
  // mask of step t needs h_t: row t of the saved states, which is the
  // previous state of step t+1, or (last step of a block, and T-1) the carry
  // hcr/hci kept from the block processed before.
  auto run_block = [&](auto h_tag, int t0, auto tail_tag) {
    constexpr int h = decltype(h_tag)::value;
    constexpr bool TAIL = decltype(tail_tag)::value;
    // the block's per-step values through LDS: lane s (< kS, the lanes above
    // repeat them) writes step s's (E = e^eta, delta, -delta / (2 pi), eta),
    // every lane reads them back (a broadcast read)
    wave_lds_fence();
    tok[lane] = make_float4(fast_exp(ev[h]), dv[h], dv[h] * kNegInv2Pi, ev[h]);
    wave_lds_fence();
    float Es[kS], Ds[kS], Rs[kS], Hs[kS];
#pragma unroll
    for (int s = 0; s < kS; ++s) {
      const float4 t4 = tok[s];
      Es[s] = t4.x;
      Ds[s] = t4.y;
      Rs[s] = t4.z;
      Hs[s] = t4.w;
    }
    float qar[kS][V], qai[kS][V], qem[kS][V];
    p1_block_transitions<IO, MODE, kS, V>(mc, Es, Ds, Rs, qar, qai, qem);
    if constexpr (RST) p1_block_resets<kS, V>(kv[h], qar, qai);
    if constexpr (GW && SUMMARY) {
      // the adjoint's map over the segment from a zero adjoint after it,
      // first step first: with P the product of conj(a) up to step t, the
      // adjoint leaving the segment is the sum of P dy_t (P <- P conj(a_t),
      // then Xr, Xi += P dy_t)
#pragma unroll
      for (int s = 0; s < kS; ++s) {
        if (TAIL && t0 + s >= t_end) break;  // wave-uniform
        float gyr[V], gyi[V];
        unpack<IO, V>(dr[h][s], gyr);
        unpack<IO, V>(di[h][s], gyi);
#pragma unroll
        for (int v = 0; v < V; ++v) {
          const float pr2 = fmaf(qar[s][v], Pr[v], qai[s][v] * Pi[v]);
          Pi[v] = fmaf(qar[s][v], Pi[v], -qai[s][v] * Pr[v]);
          Pr[v] = pr2;
          Xr[v] = fmaf(Pr[v], gyr[v], fmaf(-Pi[v], gyi[v], Xr[v]));
          Xi[v] = fmaf(Pr[v], gyi[v], fmaf(Pi[v], gyr[v], Xi[v]));
        }
      }
      return;
    }
    RawT dwr[kS], dwi[kS];          // GW: the packed dw rows
    float dxr[kS][V], dxi[kS][V];   // module: dx
    float e[2 * kS];                // e[2s], e[2s+1]: this lane's d eta, d delta of step s
#pragma unroll
    for (int s = kS - 1; s >= 0; --s) {
      const int t = t0 + s;
      if (TAIL && t >= t_end) {  // wave-uniform: no such step
        e[2 * s] = 0.0f;
        e[2 * s + 1] = 0.0f;
#pragma unroll
        for (int v = 0; v < V; ++v) { dxr[s][v] = 0.0f; dxi[s][v] = 0.0f; }
        continue;
      }
      float gyr[V], gyi[V];
      unpack<IO, V>(dr[h][s], gyr);
      unpack<IO, V>(di[h][s], gyi);
      if constexpr (!GW) {  // the relu mask: h_t > 0
        float mr[V], mi[V];
        const bool carry = s == kS - 1 || (TAIL && t == t_end - 1);  // wave-uniform
        if (carry) {
#pragma unroll
          for (int v = 0; v < V; ++v) { mr[v] = hcr[v]; mi[v] = hci[v]; }
        } else {
          unpack<IO, V>(pr[h][s + 1 < kS ? s + 1 : s], mr);
          unpack<IO, V>(pi[h][s + 1 < kS ? s + 1 : s], mi);
        }
#pragma unroll
        for (int v = 0; v < V; ++v) {
          gyr[v] = mr[v] > 0.0f ? gyr[v] : 0.0f;
          gyi[v] = mi[v] > 0.0f ? gyi[v] : 0.0f;
        }
      }
      if constexpr (SUMMARY) {  // the adjoint alone: no gradients, no stores
#pragma unroll
        for (int v = 0; v < V; ++v) {
          const float l_r = gyr[v] + Xr[v], l_i = gyi[v] + Xi[v];
          Xr[v] = fmaf(qar[s][v], l_r, qai[s][v] * l_i);
          Xi[v] = fmaf(qar[s][v], l_i, -qai[s][v] * l_r);
          const float pr2 = fmaf(qar[s][v], Pr[v], qai[s][v] * Pi[v]);  // P <- conj(a) P
          Pi[v] = fmaf(qar[s][v], Pi[v], -qai[s][v] * Pr[v]);
          Pr[v] = pr2;
        }
        continue;
      }
      float hpr[V], hpi[V], cxr[V], cxi[V];
      unpack<IO, V>(pr[h][s], hpr);
      unpack<IO, V>(pi[h][s], hpi);
      if (s == 0) {  // the state before step 0 (t = 0 only at s = 0): selects, not a branch in the block
        const bool first = t0 == 0;
#pragma unroll
        for (int v = 0; v < V; ++v) {
          hpr[v] = first ? h0r[v] : hpr[v];
          hpi[v] = first ? h0i[v] : hpi[v];
        }
      }
      if constexpr (!GW) {
        unpack<IO, V>(xr[h][s], cxr);
        unpack<IO, V>(xi[h][s], cxi);
      }
      const float E = Es[s], delta = Ds[s];
      float se = 0.0f, sd = 0.0f;
      float lrv[V], liv[V];
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const float l_r = gyr[v] + Xr[v], l_i = gyi[v] + Xi[v];
        const float xr1 = fmaf(qar[s][v], l_r, qai[s][v] * l_i);
        const float xi1 = fmaf(qar[s][v], l_i, -qai[s][v] * l_r);
        Xr[v] = xr1;
        Xi[v] = xi1;
        const float zr = fmaf(xr1, hpr[v], xi1 * hpi[v]);   // Re Z
        const float zi = fmaf(xi1, hpr[v], -xr1 * hpi[v]);  // Im Z = dphi
        const float em = qem[s][v];
        const float tt = fmaf(fmaf(em, delta, delta), zi, -zr);  // rho delta dphi - Re Z
        if constexpr (GW) {  // dw = lambda; the transition gradients alone
          lrv[v] = l_r;
          liv[v] = l_i;
          const float u = mc.nu[v] * tt;  // radial / E
          se += u;
          sd = fmaf(-em, zi, sd);
          acc[0][v] = fmaf(E, u, acc[0][v]);
          acc[1][v] += zi;
        } else {  // module: the write path too
          const float e2 = fmaf(em, em, em + em);  // em (2 + em) = expm1(-2 nu E) = rho^2 - 1
          const float sg = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(fmaf(delta, mc.pl[v], Hs[s] * mc.rl[v])));
          // one reciprocal square root gives both sqrt(Y) = Y r and 1/e2 = g2 r^2
          // (Y >= 0; the floor keeps a zero gain at zero instead of 0 * inf)
          const float Y = mc.g2[v] * e2, r = __builtin_amdgcn_rsqf(fmaxf(Y, 1e-30f));
          const float gain = Y * r * sg;
          const float tr = tanh_fast(cxr[v]), ti = tanh_fast(cxi[v]);
          float w_r = l_r, w_i = l_i;  // the write's gradient
          if constexpr (kRoundWrite<IO>) round_bf16x2(w_r, w_i);
          const float wgr = w_r * gain, wgi = w_i * gain;
          dxr[s][v] = wgr * fmaf(-tr, tr, 1.0f);
          dxi[s][v] = wgi * fmaf(-ti, ti, 1.0f);
          const float g = fmaf(wgr, tr, wgi * ti);
          // radial + g wterm = E nu (tt - g rho^2 / e2) with rho^2 / e2 = 1 + g2 r^2
          // (nu E is the transition's own product)
          const float ue = (mc.nu[v] * E) * fmaf(-g, fmaf(mc.g2[v], r * r, 1.0f), tt);
          const float gs = g * (1.0f - sg);
          se = fmaf(gs, mc.wrr_s[v], se + ue);
          sd = fmaf(-em, zi, fmaf(gs, mc.wpr_s[v], sd));
          // constant factors applied once after the sums: d nu_log's
          // -kappa sum g, d wpr's 2/pi, d wrr's 1/log16
          acc[0][v] += ue;
          acc[1][v] += zi;
          acc[2][v] += g;
          acc[3][v] = fmaf(gs, delta, acc[3][v]);
          acc[4][v] = fmaf(gs, Hs[s], acc[4][v]);
        }
      }
      if constexpr (GW) {
        dwr[s] = pack<IO, V>(lrv);
        dwi[s] = pack<IO, V>(liv);
        e[2 * s] = se * E;
      } else {
        e[2 * s] = lane_ok ? se : 0.0f;  // lanes past M: finite zeros from their zero constants, kept exact
      }
      e[2 * s + 1] = GW || lane_ok ? sd : 0.0f;
    }
    if constexpr (SUMMARY) {
      if constexpr (!GW) {
        unpack<IO, V>(pr[h][0], hcr);
        unpack<IO, V>(pi[h][0], hci);
      }
      return;
    }
    // (C) stores; the carry for the next block (in reverse time) is h_{t0-1}
    if constexpr (GW) {  // dw_re, dw_im planes
      const int64_t woff = wave_uniform(((row0 + t0) * a.M + mbase) * ESZ);
      const __amdgpu_buffer_rsrc_t rwr = make_rsrc(static_cast<char*>(a.dx) + woff, blk_h);
      const __amdgpu_buffer_rsrc_t rwi = make_rsrc(static_cast<char*>(a.dw_im) + woff, blk_h);
#pragma unroll
      for (int s = 0; s < kS; ++s) {
        if (TAIL && t0 + s >= t_end) break;
        const uint32_t o = static_cast<uint32_t>(s) * half_x;
        buf_store<RawT, CPOL_NT>(dwr[s], rwr, lane_st, o);
        buf_store<RawT, CPOL_NT>(dwi[s], rwi, lane_st, o);
      }
    } else if constexpr (!COOP) {
      const int64_t xoff = wave_uniform(((row0 + t0) * W + mbase) * ESZ);
      const __amdgpu_buffer_rsrc_t rdx = make_rsrc(static_cast<char*>(a.dx) + xoff, blk_x);
#pragma unroll
      for (int s = 0; s < kS; ++s) {
        if (TAIL && t0 + s >= t_end) break;
        const uint32_t o = static_cast<uint32_t>(s) * row_x;
        buf_store<RawT, CPOL_NT>(pack<IO, V>(dxr[s]), rdx, lane_st, o);
        buf_store<RawT, CPOL_NT>(pack<IO, V>(dxi[s]), rdx, lane_st, o + half_x);
      }
    }
    // the wave sums of the block's 2*kS per-token values: the first lane of
    // each group of G lanes holds K of them (values i = lane / G * K + k)
    wave_sums_to_leaders<2 * kS>(e);
    constexpr int K = 2 * kS >= 16 ? 2 * kS / 16 : 1, G = 64 * K / (2 * kS);
    if constexpr (COOP) {
      // Blocks go nblk-1 .. 0.  Each step below waits on memory operations
      // issued at least a block earlier, so that a block's compute hides them.
      const int kb = (t0 - t_begin) / kS;
      // reduce the block this chain owns once its records are in (tried at
      // each block's end from two blocks after it)
      if (pend < 0 && kb + 2 < nblk && (kb + 2) % a.n_mb == mb) pend = kb + 2;
      if (pend >= 0 && coop_reduce(pend, false)) pend = -1;
      coop_store_record(kb, e);
      // complete block kb + L (this block's slot) with the gradient loaded at
      // the previous block's end; load the one the next block completes
      if (kb + L < nblk) {
        coop_await(kb + L, dpn);
        coop_finish(kb + L, dpn);
      }
      if (kb >= 1 && kb + L - 1 < nblk) coop_load_grad(kb + L - 1, dpn);
      const int sl = kb % L;
#pragma unroll
      for (int s = 0; s < kS; ++s) cring[sl][s][lane] = CoopRing<IO>::put(dxr[s][0], dxi[s][0], xr[h][s], xi[h][s]);
    } else {
      // value i (d eta for even i, d delta for odd i, of step t0 + i/2) goes
      // through the resource of its plane, which covers the block's steps
      // inside the segment; the other plane's store, non-leader lanes and
      // steps past the segment are dropped (no store under a branch)
      const uint32_t nb = static_cast<uint32_t>(min(kS, t_end - t0)) * 4u;
      const int64_t o0 = wave_uniform(((static_cast<int64_t>(0) * a.n_mb + mb) * Rp + tok0 + t0) * 4);
      const int64_t o1 = wave_uniform(((static_cast<int64_t>(1) * a.n_mb + mb) * Rp + tok0 + t0) * 4);
      const __amdgpu_buffer_rsrc_t rt0 = make_rsrc(reinterpret_cast<char*>(a.part_tok) + o0, nb);
      const __amdgpu_buffer_rsrc_t rt1 = make_rsrc(reinterpret_cast<char*>(a.part_tok) + o1, nb);
      const bool lead = lane % G == 0;
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int i = lane / G * K + k;
        const uint32_t off = static_cast<uint32_t>(i >> 1) * 4u;
        const float v[1] = {e[k]};
        buffer_store_f32<1, CPOL_DEFAULT>(rt0, lead && !(i & 1) ? off : kDropOffset, v);
        buffer_store_f32<1, CPOL_DEFAULT>(rt1, lead && (i & 1) ? off : kDropOffset, v);
      }
    }
    if constexpr (!GW) {
      unpack<IO, V>(pr[h][0], hcr);
      unpack<IO, V>(pi[h][0], hci);
    }
  };

  // block k uses register buffer k & 1 (compile-time in each call, see the
  // forward).  A summary of given writes walks its segment first block first
  // (blk): the rows it read last, still in the caches when the replay starts,
  // are then the ones the replay (in reverse time) reads first.
  auto blk = [&](int k) { return GW && SUMMARY ? n_blocks - 1 - k : k; };
  auto step_block = [&](auto h_tag, int k) {
    constexpr int h = decltype(h_tag)::value;
    load_block(std::integral_constant<int, 1 - h>{}, blk(k > 0 ? k - 1 : k));
    const int t0 = t_begin + blk(k) * kS;
    if (t0 + kS <= t_end) run_block(h_tag, t0, std::false_type{});
    else run_block(h_tag, t0, std::true_type{});
  };
  int k = n_blocks - 1;
  if (k & 1) {
    load_block(std::integral_constant<int, 1>{}, blk(k));
    step_block(std::integral_constant<int, 1>{}, k);
    --k;
  } else {
    load_block(std::integral_constant<int, 0>{}, blk(k));
  }
  for (; k >= 0; k -= 2) {  // k even here
    step_block(std::integral_constant<int, 0>{}, k);
    if (k >= 1) step_block(std::integral_constant<int, 1>{}, k - 1);
  }
  if constexpr (COOP) {
    // complete the blocks still in the ring (reducing the ones this chain
    // owns on the way), then store this chain's direction sums
    for (int kc = min(L, nblk) - 1; kc >= 0; --kc) {
      float v[NV];
      coop_load_grad(kc, v);
      coop_await(kc, v);
      coop_finish(kc, v);
    }
    if (lane_ok) {
      float* p0 = a.coop_pd + static_cast<int64_t>(b) * W;                 // [0][b]: phase
      float* p1 = a.coop_pd + (static_cast<int64_t>(a.B) + b) * W;         // [1][b]: radial
      p0[m0] = ad[0];
      p1[m0] = ad[1];
      p0[a.M + m0] = ad[2];
      p1[a.M + m0] = ad[3];
    }
  }
  if constexpr (SUMMARY) {
    if (lane_ok) {
#pragma unroll
      for (int v = 0; v < V; ++v)
        *reinterpret_cast<float4*>(a.seg_sum + ((static_cast<int64_t>(b) * a.n_seg + cp.seg) * a.M + m0 + v) * 4) =
            make_float4(Pr[v], Pi[v], Xr[v], Xi[v]);
    }
  } else if (lane_ok) {
    const int64_t rows = static_cast<int64_t>(a.B) * a.n_seg, row = static_cast<int64_t>(b) * a.n_seg + cp.seg;
    constexpr int NP = GW ? 2 : 5;  // GW: nu_log and theta_log only
#pragma unroll
    for (int v = 0; v < V; ++v) {
      acc[1][v] *= mc.th[v];  // d theta_log = theta sum dphi
      if constexpr (!GW) {    // the module's constant factors (run_block)
        acc[0][v] = fmaf(-mc.kappa[v], acc[2][v], acc[0][v]);
        acc[3][v] *= kTwoOverPi;
        acc[4][v] *= kInvLog16;
      }
    }
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int v = 0; v < V; ++v)
        a.part_mode[(p * rows + row) * a.M + m0 + v] = acc[p][v];
    if (a.piped && cp.seg > 0) {  // the adjoint entering the piece before this one
#pragma unroll
      for (int v = 0; v < V; ++v)
        *reinterpret_cast<float2*>(a.seg_state +
                                   ((static_cast<int64_t>(b) * a.n_seg + cp.seg - 1) * a.M + m0 + v) * 2) =
            make_float2(Xr[v], Xi[v]);
    }
    if constexpr (GW) {  // the gradient of the initial state: conj(a_0) lambda_0
      if (t_begin == 0 && a.dh0_re) {
#pragma unroll
        for (int v = 0; v < V; ++v) {
          a.dh0_re[static_cast<int64_t>(b) * a.M + m0 + v] = Xr[v];
          a.dh0_im[static_cast<int64_t>(b) * a.M + m0 + v] = Xi[v];
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// carries across time segments
// ---------------------------------------------------------------------------
// Each segment maps the state entering it to the state leaving it, h -> P h + Q
// (forward: P the product of its transitions, Q its end state from zero;
// backward: the same for the adjoint with conj(a), in reverse time).  The
// state entering segment s is the composition of the maps of the segments
// processed before it (forward 0 .. s-1 applied to zero; backward n-1 .. s+1
// applied to dlast).  One wave per (batch row, mode): lane j takes the j-th
// segment in processing order of each group of 64, a Hillis-Steele scan over
// the lanes composes the maps, and each group's composition carries into the
// next.  The last segment processed has no map (its summary is not needed).
__global__ void __launch_bounds__(64)
mixer_seg_carry_kernel(int B, int M, int n_seg, int reverse, const float* seg_sum, const float* init_re,
                       const float* init_im, float* seg_state) {
  // i = b * M + m; neighbouring modes share the cache lines of seg_sum and
  // seg_state (8 and 16 to a line), so they run on the same XCD (one L2)
  const int i = xcd_swizzle(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x)), lane = threadIdx.x;
  const int b = i / M, m = i - b * M;
  float cr = init_re ? init_re[i] : 0.0f, ci = init_im ? init_im[i] : 0.0f;
  for (int g0 = 0; g0 < n_seg; g0 += 64) {
    const int j = g0 + lane;                      // position in processing order
    const int sg = reverse ? n_seg - 1 - j : j;   // the segment
    float pr = 1.0f, pi = 0.0f, qr = 0.0f, qi = 0.0f;  // identity past the end / for the last segment
    if (j < n_seg - 1) {
      const float4 e = *reinterpret_cast<const float4*>(seg_sum + ((static_cast<int64_t>(b) * n_seg + sg) * M + m) * 4);
      pr = e.x; pi = e.y; qr = e.z; qi = e.w;
    }
    // inclusive scan: lane j holds map_j o ... o map_g0
#pragma unroll
    for (int d = 1; d < 64; d *= 2) {
      const float ppr = __shfl_up(pr, d), ppi = __shfl_up(pi, d);
      const float pqr = __shfl_up(qr, d), pqi = __shfl_up(qi, d);
      if (lane >= d) {  // (P, Q) o (Pp, Qp) = (P Pp, P Qp + Q)
        const float nqr = fmaf(pr, pqr, fmaf(-pi, pqi, qr));
        const float nqi = fmaf(pr, pqi, fmaf(pi, pqr, qi));
        const float npr = fmaf(pr, ppr, -pi * ppi);
        const float npi = fmaf(pr, ppi, pi * ppr);
        pr = npr; pi = npi; qr = nqr; qi = nqi;
      }
    }
    // the state entering segment sg: the maps before it (exclusive) applied to the carry
    const float epr = __shfl_up(pr, 1), epi = __shfl_up(pi, 1), eqr = __shfl_up(qr, 1), eqi = __shfl_up(qi, 1);
    float hr = cr, hi = ci;
    if (lane > 0) {
      hr = fmaf(epr, cr, fmaf(-epi, ci, eqr));
      hi = fmaf(epr, ci, fmaf(epi, cr, eqi));
    }
    if (j < n_seg)
      *reinterpret_cast<float2*>(seg_state + ((static_cast<int64_t>(b) * n_seg + sg) * M + m) * 2) = make_float2(hr, hi);
    // the carry into the next group: the whole group's composition
    const float lpr = __shfl(pr, 63), lpi = __shfl(pi, 63), lqr = __shfl(qr, 63), lqi = __shfl(qi, 63);
    const float ncr = fmaf(lpr, cr, fmaf(-lpi, ci, lqr));
    ci = fmaf(lpr, ci, fmaf(lpi, cr, lqi));
    cr = ncr;
  }
}

__global__ void fill_zero_f32_kernel(float* p, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) p[i] = 0.0f;
}
// p[0 .. 4 n4) = v in 16-byte stores, and the first thread also sets
// head[0 .. n_head) = head_v (the one-launch backward's error words)
__global__ void fill_u32x4_kernel(uint4* p, int64_t n4, uint32_t v, uint32_t* head, int n_head, uint32_t head_v) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < n4) p[i] = make_uint4(v, v, v, v);
  if (i == 0)
    for (int k = 0; k < n_head; ++k) head[k] = head_v;
}

// ---------------------------------------------------------------------------
// controls backward: dx += dp0 u_phase + dp1 u_radial (in place), direction
// gradient partials per row block
// ---------------------------------------------------------------------------
// dp1 = d eta * log16 (1 - tanh^2 p1) = d eta * log16 (1 - (eta/log16)^2),
// dp0 = d delta * pi/2 (1 - (delta/(pi/2))^2).  A workgroup: 2048 columns (8
// per thread) of the row blocks blockIdx.y, blockIdx.y + gridDim.y, ... of
// `rows` rows each; its partial direction gradients go to partial row
// blockIdx.y.
template <typename IO>
__global__ void __launch_bounds__(256)
ctrl_bwd_kernel(int64_t R, int W, int rows, const void* x, const float* pdir, const float* rdir,
                const float* eta, const float* delta, const float* deta, const float* ddelta,
                void* dx, float* pd, float* pbias, int64_t T, int64_t t0, int64_t L, int rb0, int n_rb) {
  const int c = (blockIdx.x * 256 + threadIdx.x) * 8;
  const bool col_ok = c < W;
  const int cc = col_ok ? c : 0;
  float u0[8], u1[8], a0[8], a1[8];
  *reinterpret_cast<float4*>(u0) = *reinterpret_cast<const float4*>(pdir + cc);
  *reinterpret_cast<float4*>(u0 + 4) = *reinterpret_cast<const float4*>(pdir + cc + 4);
  *reinterpret_cast<float4*>(u1) = *reinterpret_cast<const float4*>(rdir + cc);
  *reinterpret_cast<float4*>(u1 + 4) = *reinterpret_cast<const float4*>(rdir + cc + 4);
#pragma unroll
  for (int i = 0; i < 8; ++i) { a0[i] = 0.0f; a1[i] = 0.0f; }
  float b0 = 0.0f, b1 = 0.0f;
  // rows in groups of kG: every load of the group is issued before any of
  // its arithmetic (rows past r1 re-read row r1-1 and contribute nothing)
  constexpr int kG = 4;
  for (int64_t r0 = static_cast<int64_t>(blockIdx.y) * rows; r0 < R; r0 += static_cast<int64_t>(gridDim.y) * rows) {
    const int64_t r1 = r0 + rows < R ? r0 + rows : R;
    // row r of deta, ddelta is row r + da of x, dx, eta, delta: a time piece
    // is B runs of L rows from step t0 of each batch row (L a multiple of
    // `rows`, so a workgroup's rows stay in one run); otherwise L = T = R,
    // t0 = 0 and da = 0
    const int64_t da = (r0 / L) * T + t0 + (r0 % L) - r0;
    auto load8 = [&](const void* base, int64_t row, float (&o)[8]) {
      if constexpr (sizeof(IO) == 2) {
        unpack<bf16, 8>(load_raw_nt<bf16, 8>(base, row * W + cc), o);
      } else {
        float t[4];
        unpack<float, 4>(load_raw_nt<float, 4>(base, row * W + cc), t);
        for (int i = 0; i < 4; ++i) o[i] = t[i];
        unpack<float, 4>(load_raw_nt<float, 4>(base, row * W + cc + 4), t);
        for (int i = 0; i < 4; ++i) o[4 + i] = t[i];
      }
    };
    for (int64_t r = r0; r < r1; r += kG) {
      float xv[kG][8], gv[kG][8], dp0[kG], dp1[kG];
#pragma unroll
      for (int k = 0; k < kG; ++k) {
        const int64_t rr = r + k < r1 ? r + k : r1 - 1;
        load8(x, rr + da, xv[k]);
        load8(dx, rr + da, gv[k]);
      }
#pragma unroll
      for (int k = 0; k < kG; ++k) {
        const int64_t rr = r + k < r1 ? r + k : r1 - 1;
        const float e = eta[rr + da] * kInvLog16, d = delta[rr + da] * kTwoOverPi;
        const bool live = r + k < r1;
        dp1[k] = live ? deta[rr] * kLog16 * fmaf(-e, e, 1.0f) : 0.0f;
        dp0[k] = live ? ddelta[rr] * kHalfPi * fmaf(-d, d, 1.0f) : 0.0f;
        b0 += dp0[k];
        b1 += dp1[k];
      }
#pragma unroll
      for (int k = 0; k < kG; ++k) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          gv[k][i] = fmaf(dp0[k], u0[i], fmaf(dp1[k], u1[i], gv[k][i]));
          a0[i] = fmaf(dp0[k], xv[k][i], a0[i]);
          a1[i] = fmaf(dp1[k], xv[k][i], a1[i]);
        }
      }
      if (col_ok) {
#pragma unroll
        for (int k = 0; k < kG; ++k) {
          if (r + k >= r1) break;  // wave-uniform
          const int64_t rr = r + k + da;
          if constexpr (sizeof(IO) == 2) {
            store_raw_nt<bf16, 8>(dx, rr * W + c, pack<bf16, 8>(gv[k]));
          } else {
            float t[4];
            for (int i = 0; i < 4; ++i) t[i] = gv[k][i];
            store_raw_nt<float, 4>(dx, rr * W + c, pack<float, 4>(t));
            for (int i = 0; i < 4; ++i) t[i] = gv[k][4 + i];
            store_raw_nt<float, 4>(dx, rr * W + c + 4, pack<float, 4>(t));
          }
        }
      }
    }
  }  // row blocks
  if (col_ok) {
    // partial row rb0 + blockIdx.y of the [2][n_rb][W] partials
    float* o0 = pd + (static_cast<int64_t>(rb0) + blockIdx.y) * W + c;
    float* o1 = pd + (static_cast<int64_t>(n_rb) + rb0 + blockIdx.y) * W + c;
    *reinterpret_cast<float4*>(o0) = *reinterpret_cast<const float4*>(a0);
    *reinterpret_cast<float4*>(o0 + 4) = *reinterpret_cast<const float4*>(a0 + 4);
    *reinterpret_cast<float4*>(o1) = *reinterpret_cast<const float4*>(a1);
    *reinterpret_cast<float4*>(o1 + 4) = *reinterpret_cast<const float4*>(a1 + 4);
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    pbias[rb0 + blockIdx.y] = b0;
    pbias[n_rb + rb0 + blockIdx.y] = b1;
  }
}

}  // namespace mix
}  // namespace sparc

// ===========================================================================
// host side
// ===========================================================================
namespace {
using namespace sparc::mix;

sparc_status fail(sparc_status s, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
sparc_status fail(sparc_status s, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(sparc::error_buffer(), 512, fmt, ap);
  va_end(ap);
  return s;
}
bool al(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Modes per lane of the forward (0: automatic) and of the backward.
#ifndef SPARC_MIXER_FWD_V
#define SPARC_MIXER_FWD_V 0
#endif
#ifndef SPARC_MIXER_BWD_V
#define SPARC_MIXER_BWD_V 0
#endif
// Forward: 2 when that leaves at least 1280 chains (1.25 waves per SIMD of the
// 256-CU MI355X), else 1 (twice the chains).  Measured at B=8, M=16384 (1024
// chains of 2): 1 mode per lane 2.3 ms against 2.8 ms; at B=16, M=12288 (1536
// chains of 2): 2 modes 1.4 ms against 1.5 ms.  The forward is VALU-bound:
// more resident waves hide the latency of its dependent arithmetic.  (Both
// shapes now take the wide kernel.)  Also 2 when one mode per lane would be
// split into time segments anyway: the P1 forward at B=1, T=65536, M=2048
// 0.443 -> 0.405 ms, at B=2, T=16384, M=8192 0.84 -> 0.77 ms, the module
// step at B=1, T=65536, width 2048 1.11 -> 1.08 ms.
// Backward (module): 1, or 2 when one mode per lane would be split into time
// segments anyway (B=1, T=65536, width 2048: 1.08 -> 1.05-1.06 ms per step);
// with many chains 2 was slower (3.75 -> 3.87-3.95 ms at B=8, width 32768).
// The P1 scan's backward (writes given) with two modes per lane: 1.58-1.59 ->
// 1.46-1.49 ms at B=8, T=4096, M=16384 (1024 waves), faster at every shape
// measured.
#ifndef SPARC_P1_BWD_V
#define SPARC_P1_BWD_V 2
#endif
int mixer_v(int64_t B, int64_t T, int64_t M, int direction, bool gw);

// Time segments.  One wave per chain (batch row x 64 V modes) walks its
// whole sequence, so with fewer chains than SIMDs most of the GPU idles.
// Then the sequence is split into n_seg segments of t_seg steps (a multiple
// of 8, at least kMinSegSteps) so that about two waves per SIMD run: a
// summary pass gives each segment's map (P, Q), a carry kernel composes them
// into the state entering every segment, and the full pass replays each
// segment from its entering state.  This costs a second pass over the
// transitions (and, forward, the writes), paid for by the occupancy.
#ifndef SPARC_MIXER_SEG_CHAINS
#define SPARC_MIXER_SEG_CHAINS 1024
#endif
constexpr int64_t kSegChains = SPARC_MIXER_SEG_CHAINS;  // segment below this many chains
#ifndef SPARC_MIXER_SEG_TARGET
#define SPARC_MIXER_SEG_TARGET 4096
#endif
#ifndef SPARC_MIXER_SEG_MIN
#define SPARC_MIXER_SEG_MIN 128
#endif
constexpr int64_t kSegTarget = SPARC_MIXER_SEG_TARGET;  // waves to aim for
constexpr int64_t kMinSegSteps = SPARC_MIXER_SEG_MIN;
int mixer_v(int64_t B, int64_t T, int64_t M, int direction, bool gw) {
  const int fixed = direction == 0 ? SPARC_MIXER_FWD_V : gw ? SPARC_P1_BWD_V : SPARC_MIXER_BWD_V;
  if (fixed == 1 || M % 2) return 1;
  if (fixed == 2) return 2;
  const int64_t chains1 = B * ((M + 63) / 64), chains2 = B * ((M + 127) / 128);
  const bool segmented = chains1 < kSegChains && T >= 2 * kMinSegSteps;  // with one mode per lane
  if (direction == 1) return segmented ? 2 : 1;
  return chains2 >= 1280 || segmented ? 2 : 1;
}
void choose_segments(int64_t B, int64_t T, int n_mb, int& n_seg, int& t_seg) {
  n_seg = 1;
  t_seg = static_cast<int>(T > 0 ? T : 1);
  const int64_t chains = B * n_mb;
  if (chains >= kSegChains || T < 2 * kMinSegSteps) return;
  int64_t n = std::min((kSegTarget + chains - 1) / chains, T / kMinSegSteps);
  if (n < 2) return;
  int64_t len = (T + n - 1) / n;
  len = (len + 7) / 8 * 8;
  n = (T + len - 1) / len;
  if (n < 2) return;
  n_seg = static_cast<int>(n);
  t_seg = static_cast<int>(len);
}

// The module backward without time segments runs in time pieces: the
// controls backward of piece p then runs on a second stream while the mixer
// backward works on piece p - 1.  The most pieces, up to kPieces, whose
// length is a multiple of kCtrlBwdRows (no pieces when T allows none).
// Module fwd+bwd, bf16, against no pieces: B=8 T=4096 width 32768 5.59 ->
// 5.38 ms with at most 4 pieces, 5.24 with 8, 5.35 with 16; B=16 T=2048
// width 24576 4.21 -> 3.92 (4), 3.96 (8), 4.15 (16, pieces of 128 steps).
#ifndef SPARC_MIXER_BWD_PIECES
#define SPARC_MIXER_BWD_PIECES 8
#endif
constexpr int kPieces = SPARC_MIXER_BWD_PIECES;

struct Layout {
  bool piped = false;
  int V = 1, n_mb = 0, n_rb = 0, n_rb_piece = 0, n_seg = 1, t_seg = 1;
  int64_t R = 0;
  size_t consts = 0, part_tok = 0, tok = 0, part_mode = 0, pd = 0, pbias = 0, seg_sum = 0, seg_state = 0, total = 0;
};

// gw: the P1 scan with the writes given (no controls, two per-mode gradients);
// pieces: the module backward in time pieces where the shape allows
Layout layout(int64_t B, int64_t T, int64_t M, int direction, bool gw = false, bool pieces = false) {
  Layout l;
  l.V = mixer_v(B, T, M, direction, gw);
  l.n_mb = static_cast<int>((M + 64 * l.V - 1) / (64 * l.V));
  choose_segments(B, T, l.n_mb, l.n_seg, l.t_seg);
  l.R = B * T;
  l.n_rb = static_cast<int>(std::min<int64_t>((l.R + kCtrlBwdRows - 1) / kCtrlBwdRows, kMaxRowBlocks));
  int np = kPieces;
  while (np > 1 && T % (static_cast<int64_t>(np) * kCtrlBwdRows) != 0) np /= 2;
  if (pieces && np > 1 && T > 0 && direction == 1 && !gw && l.n_seg == 1 && l.V == 1) {
    l.piped = true;
    l.n_seg = np;
    l.t_seg = static_cast<int>(T / np);
    l.n_rb_piece = static_cast<int>(std::min<int64_t>(B * l.t_seg / kCtrlBwdRows, kMaxRowBlocks));
    l.n_rb = np * l.n_rb_piece;
  }
  auto up = [](size_t n) { return (n + 255) / 256 * 256; };
  size_t off = 256;
  l.consts = off;
  off += up(static_cast<size_t>(M) * kConsts * 4);
  if (l.n_seg > 1) {
    l.seg_sum = off;
    if (!l.piped) off += up(static_cast<size_t>(B) * l.n_seg * M * 4 * 4);
    l.seg_state = off;
    off += up(static_cast<size_t>(B) * l.n_seg * M * 2 * 4);
  }
  if (direction == 1 && gw) {
    l.part_tok = off;
    off += up(static_cast<size_t>(2) * l.n_mb * l.R * 4);
    l.part_mode = off;
    off += up(static_cast<size_t>(2) * B * l.n_seg * M * 4);
  } else if (direction == 1) {
    l.part_tok = off;
    off += up(static_cast<size_t>(2) * l.n_mb * l.R * 4);
    l.tok = off;
    off += up(static_cast<size_t>(2) * l.R * 4);
    l.part_mode = off;
    off += up(static_cast<size_t>(5) * B * l.n_seg * M * 4);
    l.pd = off;
    off += up(static_cast<size_t>(2) * l.n_rb * 2 * M * 4);
    l.pbias = off;
    off += up(static_cast<size_t>(2) * l.n_rb * 4);
  }
  l.total = off;
  return l;
}

sparc_status check_shape(int64_t B, int64_t T, int64_t M, int32_t io) {
  if (B <= 0 || T < 0 || M <= 0) return fail(SPARC_EINVAL, "mixer: B > 0, T >= 0, M > 0 required");
  if (M % 4) return fail(SPARC_EINVAL, "mixer: modes must be a multiple of 4");
  if (io != SPARC_F32 && io != SPARC_BF16) return fail(SPARC_EINVAL, "mixer: io_dtype");
  if (M > (1 << 24) || B * T > (int64_t(1) << 40) || B * T * 2 * M > (int64_t(1) << 46) || B > INT32_MAX ||
      T > INT32_MAX)
    return fail(SPARC_EINVAL, "mixer: shape too large");
  return SPARC_OK;
}

// the forward over n_segs segments from a.seg_lo (SUMMARY: the maps only)
template <typename IO, int V, bool SUMMARY, int MODE>
void launch_fwd(const Args& a, int n_segs, hipStream_t st) {
  const dim3 g(static_cast<unsigned>(a.B) * a.n_mb * static_cast<unsigned>(n_segs));
  hipLaunchKernelGGL((mixer_fwd_kernel<IO, V, SUMMARY, MODE>), g, dim3(64), 0, st, a);
}
template <typename IO, int V, int MODE = kModule>
void run_fwd(const Args& a, hipStream_t st) {
  if (a.n_seg > 1) {  // maps of segments 0 .. n-2, then the entering states (from h0, if any)
    // (the summaries read the writes only: kRelu shares the kPlanes kernel)
    launch_fwd<IO, V, true, (MODE & 3) == kModule ? kModule : (kPlanes | (MODE & kReset))>(a, a.n_seg - 1, st);
    hipLaunchKernelGGL(mixer_seg_carry_kernel, dim3(static_cast<unsigned>(a.B) * a.M), dim3(64), 0, st, a.B, a.M,
                       a.n_seg, 0, a.seg_sum, a.h0_re, a.h0_im, a.seg_state);
  }
  launch_fwd<IO, V, false, MODE>(a, a.n_seg, st);
}
// Steps per block of the backward.  8-step blocks prefetch twice as far
// ahead; the module backward then needs about 240 VGPRs (two waves per SIMD
// instead of three at 4 steps), so it takes them only when its grid leaves
// at most two waves per SIMD of the 1024 (B=8, T=4096, width 32768: 3.85 ->
// 3.75 ms; B=16, T=2048, width 24576, 3072 waves: 2.77 -> 2.81 ms with 8).
// The P1 scan (writes given) fits 8-step blocks in about 147 VGPRs: 1.61 ->
// 1.52 ms at B=8, T=4096, M=16384, and faster with time segments too.  At two
// modes per lane and without time segments, 16-step blocks at one wave per
// SIMD were faster while the kernel was bound by its VALU work (B=8, T=4096,
// M=16384: 1.43 -> 1.39 ms); with the transitions' hardware sine and cosine
// and the transition gradients taken from conj(a) lambda it streams at its
// access pattern's rate (the same time with the arithmetic stubbed out), and
// 8-step blocks at two waves per SIMD are 2 % faster (1.29 -> 1.26 ms); with
// the later cuts 4-step blocks are faster again (1.29-1.31 -> 1.24-1.26 ms;
// 2 steps 1.58-1.62, 16 steps 1.31-1.33).  With time segments the P1
// backward keeps 8-step blocks (4 measured the same).
#ifndef SPARC_MIXER_BWD_P1_S
#define SPARC_MIXER_BWD_P1_S 4
#endif
#ifndef SPARC_MIXER_BWD_S
#define SPARC_MIXER_BWD_S 4
#endif
#ifndef SPARC_MIXER_BWD_LONG_S
#define SPARC_MIXER_BWD_LONG_S 8
#endif
constexpr unsigned kBwdLongWaves = 2048;  // the module's 8-step blocks up to this grid
template <typename IO, int V, bool SUMMARY, int MODE>
void launch_bwd(const Args& a, int n_segs, hipStream_t st) {
  const unsigned waves = static_cast<unsigned>(a.B) * a.n_mb * static_cast<unsigned>(n_segs);
  const dim3 g(waves);
  if constexpr ((MODE & 3) == kModule && V == 1) {
    if (waves <= kBwdLongWaves) {
      hipLaunchKernelGGL((mixer_bwd_kernel<IO, V, SPARC_MIXER_BWD_LONG_S, SUMMARY, MODE>), g, dim3(64), 0, st, a);
      return;
    }
  }
  if constexpr ((MODE & 3) != kModule) {
    if (a.n_seg == 1) {  // no time segments; fp32 keeps 16-step blocks at one wave per SIMD (8 would spill)
      constexpr int S = sizeof(IO) == 2 ? SPARC_MIXER_BWD_P1_S : 16;
      hipLaunchKernelGGL((mixer_bwd_kernel<IO, V, S, SUMMARY, MODE>), g, dim3(64), 0, st, a);
      return;
    }
  }
  constexpr int S = (MODE & 3) == kModule ? SPARC_MIXER_BWD_S : SPARC_MIXER_BWD_LONG_S;
  hipLaunchKernelGGL((mixer_bwd_kernel<IO, V, S, SUMMARY, MODE>), g, dim3(64), 0, st, a);
}
template <typename IO, int V, int MODE = kModule>
void run_bwd(const Args& a, hipStream_t st) {
  if (a.n_seg > 1) {  // maps of segments n-1 .. 1 (reverse time), then the entering adjoints
    Args s = a;
    s.seg_lo = 1;
    launch_bwd<IO, V, true, MODE>(s, a.n_seg - 1, st);
    hipLaunchKernelGGL(mixer_seg_carry_kernel, dim3(static_cast<unsigned>(a.B) * a.M), dim3(64), 0, st, a.B, a.M,
                       a.n_seg, 1, a.seg_sum, a.dlast_re, a.dlast_im, a.seg_state);
  }
  launch_bwd<IO, V, false, MODE>(a, a.n_seg, st);
}

// The module forward takes the wide kernel (4 modes per lane, four helper
// waves, 8-step blocks) with at least kWideChains chains of 256 modes and no
// time segments.  Forward + backward, measured against the one- and two-mode
// kernels (bf16): B=8 T=4096 width 32768 (512 chains) 5.89 -> 5.46 ms;
// B=16 T=2048 width 24576 (768) 4.19 -> 4.04 ms; B=32 T=1024 width 16384
// (1024) 2.80 -> 2.81 ms; below 512 chains mixed (B=8 T=2048 width 16384 1.68
// -> 1.64 ms, B=4 T=4096 width 32768 3.73 -> 3.91 ms, B=6 4.88 -> 4.94 ms):
// the forward itself is faster at every one of these shapes, the backward
// launched after it is not always as fast.  2 helper waves were slower, 8
// helper waves or 4-step blocks the same.
#ifndef SPARC_MIXER_WIDE
#define SPARC_MIXER_WIDE 1
#endif
#ifndef SPARC_MIXER_WIDE_HELPERS
#define SPARC_MIXER_WIDE_HELPERS 4
#endif
#ifndef SPARC_MIXER_WIDE_S
#define SPARC_MIXER_WIDE_S 8
#endif
#ifndef SPARC_MIXER_WIDE_CHAINS
#define SPARC_MIXER_WIDE_CHAINS 512
#endif
constexpr int kWideHelpers = SPARC_MIXER_WIDE_HELPERS;
constexpr int kWideS = SPARC_MIXER_WIDE_S;
constexpr int64_t kWideChains = SPARC_MIXER_WIDE_CHAINS;
// The module forward above 1024 such chains keeps the two-mode kernel (B=32,
// T=1024, width 32768, 2048 chains: 5.21-5.23 against 5.30-5.43 ms per step;
// at 1024 chains the two are even); the P1 forward takes the wide kernel at
// every count measured (up to 2048 chains).
constexpr int64_t kWideChainsMaxModule = 1024;
bool fwd_wide(const Layout& l, int64_t batch, int64_t modes, bool module = false) {
  const int64_t chains = batch * ((modes + 255) / 256);
  return SPARC_MIXER_WIDE && l.n_seg == 1 && modes % 4 == 0 && chains >= kWideChains &&
         (!module || chains <= kWideChainsMaxModule);
}

// the wide forward (a.n_mb: blocks of 256 modes)
template <int MODE>
void run_fwd_wide(const Args& a, bool bf, hipStream_t st) {
  const dim3 g(static_cast<unsigned>(a.B) * static_cast<unsigned>(a.n_mb)), blk(64 * (kWideHelpers + 1));
  if (bf) hipLaunchKernelGGL((mixer_fwd_wide_kernel<sparc::bf16, kWideHelpers, kWideS, MODE>), g, blk, 0, st, a);
  else hipLaunchKernelGGL((mixer_fwd_wide_kernel<float, kWideHelpers, kWideS, MODE>), g, blk, 0, st, a);
}

// The scan and its backward with the controls given; the per-mode constants
// are built in the workspace first.  Shapes, pointers and the workspace are
// checked by the callers.
sparc_status scan_forward_impl(const Layout& l, int64_t batch, int64_t length, int64_t modes, int32_t io_dtype,
                               const void* x, const float* eta, const float* delta, const float* nu_log,
                               const float* theta_log, const float* write_log_gain,
                               const float* write_phase_response, const float* write_radial_response, void* y,
                               void* h_re, void* h_im, float* last_re, float* last_im, char* ws, hipStream_t st) {
  const int M = static_cast<int>(modes);
  float* consts = reinterpret_cast<float*>(ws + l.consts);
  hipLaunchKernelGGL(mixer_prepare_kernel, dim3(static_cast<unsigned>((M + 255) / 256)), dim3(256), 0, st, M, nu_log,
                     theta_log, write_log_gain, write_phase_response, write_radial_response, consts);
  if (length == 0) {  // the state stays 0
    if (last_re) {
      const int64_t n = batch * modes;
      const dim3 g(static_cast<unsigned>((n + 255) / 256));
      hipLaunchKernelGGL(fill_zero_f32_kernel, g, dim3(256), 0, st, last_re, n);
      hipLaunchKernelGGL(fill_zero_f32_kernel, g, dim3(256), 0, st, last_im, n);
    }
  } else {
    Args a{};
    a.B = static_cast<int>(batch);
    a.T = static_cast<int>(length);
    a.M = M;
    a.n_mb = l.n_mb;
    a.x = x; a.consts = consts; a.eta = eta; a.delta = delta;
    a.y = y; a.h_re = h_re; a.h_im = h_im; a.last_re = last_re; a.last_im = last_im;
    a.n_seg = l.n_seg; a.t_seg = l.t_seg; a.seg_lo = 0;
    a.seg_sum = reinterpret_cast<float*>(ws + l.seg_sum);
    a.seg_state = reinterpret_cast<float*>(ws + l.seg_state);
    if (fwd_wide(l, batch, modes, true)) {
      a.n_mb = static_cast<int>((modes + 255) / 256);
      run_fwd_wide<kModule>(a, io_dtype == SPARC_BF16, st);
    } else if (io_dtype == SPARC_BF16) {
      if (l.V == 2) run_fwd<sparc::bf16, 2>(a, st); else run_fwd<sparc::bf16, 1>(a, st);
    } else {
      if (l.V == 2) run_fwd<float, 2>(a, st); else run_fwd<float, 1>(a, st);
    }
  }
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? SPARC_OK : fail(SPARC_EHIP, "mixer scan forward: %s", hipGetErrorString(e));
}

sparc_status scan_backward_impl(const Layout& l, int64_t batch, int64_t length, int64_t modes, int32_t io_dtype,
                                const void* x, const float* eta, const float* delta, const float* nu_log,
                                const float* theta_log, const float* write_log_gain,
                                const float* write_phase_response, const float* write_radial_response,
                                const void* h_re, const void* h_im, const void* dy, const float* dlast_re,
                                const float* dlast_im, void* dx, float* deta, float* ddelta, float* dnu_log,
                                float* dtheta_log, float* dwrite_log_gain, float* dwrite_phase_response,
                                float* dwrite_radial_response, char* ws, sparc_stream_t stream) {
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int M = static_cast<int>(modes);
  float* consts = reinterpret_cast<float*>(ws + l.consts);
  float* part_tok = reinterpret_cast<float*>(ws + l.part_tok);
  float* part_mode = reinterpret_cast<float*>(ws + l.part_mode);
  float* outs[5] = {dnu_log, dtheta_log, dwrite_log_gain, dwrite_phase_response, dwrite_radial_response};
  hipLaunchKernelGGL(mixer_prepare_kernel, dim3(static_cast<unsigned>((M + 255) / 256)), dim3(256), 0, st, M, nu_log,
                     theta_log, write_log_gain, write_phase_response, write_radial_response, consts);
  if (length == 0) {
    const dim3 gm(static_cast<unsigned>((M + 255) / 256));
    for (float* o : outs) hipLaunchKernelGGL(fill_zero_f32_kernel, gm, dim3(256), 0, st, o, static_cast<int64_t>(M));
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? SPARC_OK : fail(SPARC_EHIP, "mixer scan backward: %s", hipGetErrorString(e));
  }
  Args a{};
  a.B = static_cast<int>(batch);
  a.T = static_cast<int>(length);
  a.M = M;
  a.n_mb = l.n_mb;
  a.x = x; a.consts = consts; a.eta = eta; a.delta = delta;
  a.h_re = const_cast<void*>(h_re); a.h_im = const_cast<void*>(h_im);
  a.dy = dy; a.dlast_re = dlast_re; a.dlast_im = dlast_im; a.dx = dx;
  a.part_tok = part_tok; a.part_mode = part_mode;
  a.n_seg = l.n_seg; a.t_seg = l.t_seg; a.seg_lo = 0;
  a.seg_sum = reinterpret_cast<float*>(ws + l.seg_sum);
  a.seg_state = reinterpret_cast<float*>(ws + l.seg_state);
  if (io_dtype == SPARC_BF16) {
    if (l.V == 2) run_bwd<sparc::bf16, 2>(a, st); else run_bwd<sparc::bf16, 1>(a, st);
  } else {
    if (l.V == 2) run_bwd<float, 2>(a, st); else run_bwd<float, 1>(a, st);
  }
  // d eta, d delta per token: the sums over the mode blocks of part_tok [2][n_mb][R]
  {
    const float* in[2] = {part_tok, part_tok + static_cast<int64_t>(l.n_mb) * l.R};
    float* out[2] = {deta, ddelta};
    if (sparc_status s = sparc::column_sums(l.n_mb, l.R, 2, in, out, stream)) return s;
  }
  const int64_t prow = batch * l.n_seg;  // one partial row per (batch row, segment)
  {
    const float* in[5];
    for (int p = 0; p < 5; ++p) in[p] = part_mode + static_cast<int64_t>(p) * prow * modes;
    if (sparc_status s = sparc::column_sums(prow, modes, 5, in, outs, stream)) return s;
  }
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? SPARC_OK : fail(SPARC_EHIP, "mixer scan backward: %s", hipGetErrorString(e));
}

bool params_ok(const float* a, const float* b, const float* c, const float* d, const float* e) {
  return a && b && c && d && e;
}

// The controls' direction gradients from their row-block partials: columns
// 0..W-1 from pd [2][n_rb][W] (phase, radial), the bias entries (column W)
// from pbias [2][n_rb]; two launches of paired column sums.
sparc_status direction_sums(int64_t n_rb, int64_t W, const float* pd, const float* pbias, float* dphase,
                            float* dradial, sparc_stream_t stream) {
  {
    const float* in[2] = {pd, pd + n_rb * W};
    float* out[2] = {dphase, dradial};
    if (sparc_status s = sparc::column_sums(n_rb, W, 2, in, out, stream)) return s;
  }
  const float* in[2] = {pbias, pbias + n_rb};
  float* out[2] = {dphase + W, dradial + W};
  return sparc::column_sums(n_rb, 1, 2, in, out, stream);
}

#ifndef SPARC_P1_FUSED
#define SPARC_P1_FUSED 1
#endif
}  // namespace

// ---------------------------------------------------------------------------
// the P1 scan with the writes given (sparc_scan_forward / _backward, G = 1)
// ---------------------------------------------------------------------------
namespace sparc {
using namespace sparc::mix;

sparc_status seg_carry(int64_t B, int64_t M, int n_seg, int reverse, const float* seg_sum, const float* init_re,
                       const float* init_im, float* seg_state, sparc_stream_t stream) {
  if (B <= 0 || M <= 0 || n_seg < 1 || B * M > INT32_MAX) return fail(SPARC_EINVAL, "seg_carry: shape");
  hipLaunchKernelGGL(mixer_seg_carry_kernel, dim3(static_cast<unsigned>(B * M)), dim3(64), 0,
                     reinterpret_cast<hipStream_t>(stream), static_cast<int>(B), static_cast<int>(M), n_seg, reverse,
                     seg_sum, init_re, init_im, seg_state);
  return SPARC_OK;  // a launch error stays for the caller's hipGetLastError
}

bool p1_fused_shape(const sparc_scan_desc* d) {
  constexpr int32_t forced = SPARC_FLAG_ALGO_LOOKBACK | SPARC_FLAG_ALGO_CHAIN | SPARC_FLAG_ALGO_SERIAL;
  if (!SPARC_P1_FUSED || !d || d->transition != SPARC_TRANSITION_P1 || d->groups != 1) return false;
  if (d->flags & forced) return false;
  if (d->gate_dtype != SPARC_F32) return false;
  return check_shape(d->batch, d->length, d->modes, d->io_dtype) == SPARC_OK;
}

size_t p1_fused_workspace_bytes(const sparc_scan_desc* d, int direction) {
  if (!p1_fused_shape(d)) return 0;
  return layout(d->batch, d->length, d->modes, direction, true).total;
}

// the launches of one chain mode for the I/O type and modes per lane
template <int MODE>
void run_fwd_mode(const Args& a, bool bf, int V, hipStream_t st) {
  if (bf) {
    if (V == 2) run_fwd<sparc::bf16, 2, MODE>(a, st); else run_fwd<sparc::bf16, 1, MODE>(a, st);
  } else {
    if (V == 2) run_fwd<float, 2, MODE>(a, st); else run_fwd<float, 1, MODE>(a, st);
  }
}
template <int MODE>
void run_bwd_mode(const Args& a, bool bf, int V, hipStream_t st) {
  if (bf) {
    if (V == 2) run_bwd<sparc::bf16, 2, MODE>(a, st); else run_bwd<sparc::bf16, 1, MODE>(a, st);
  } else {
    if (V == 2) run_bwd<float, 2, MODE>(a, st); else run_bwd<float, 1, MODE>(a, st);
  }
}

sparc_status p1_fused_forward(const sparc_scan_desc* d, const float* eta, const float* delta,
                              const float* nu_log, const float* theta_log, const void* w_re, const void* w_im,
                              const float* h0_re, const float* h0_im, const int32_t* segment_pos, void* y_re,
                              void* y_im, float* chunk_state, void* workspace, size_t workspace_bytes,
                              sparc_stream_t stream) {
  if (!p1_fused_shape(d) || d->length <= 0) return fail(SPARC_EINVAL, "p1 fused forward: shape");
  const Layout l = layout(d->batch, d->length, d->modes, 0, true);
  if (workspace_bytes < l.total) return fail(SPARC_EWORKSPACE, "workspace too small: %zu < %zu", workspace_bytes, l.total);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  const int M = static_cast<int>(d->modes);
  float* consts = reinterpret_cast<float*>(ws + l.consts);
  hipLaunchKernelGGL(mixer_prepare_kernel, dim3(static_cast<unsigned>((M + 255) / 256)), dim3(256), 0, st, M, nu_log,
                     theta_log, nullptr, nullptr, nullptr, consts);
  const bool relu = (d->flags & SPARC_FLAG_RELU_OUTPUT) != 0;
  Args a{};
  a.B = static_cast<int>(d->batch);
  a.T = static_cast<int>(d->length);
  a.M = M;
  a.n_mb = l.n_mb;
  a.consts = consts; a.eta = eta; a.delta = delta;
  a.w_re = w_re; a.w_im = w_im; a.h0_re = h0_re; a.h0_im = h0_im; a.chunk_state = chunk_state;
  a.segpos = segment_pos;
  a.reset_first = (d->flags & SPARC_FLAG_RESET_FIRST) != 0;
  const bool reset = segment_pos != nullptr || a.reset_first;
  if (relu) {
    a.y = y_re;
  } else {
    a.h_re = y_re;
    a.h_im = y_im;
  }
  a.n_seg = l.n_seg; a.t_seg = l.t_seg; a.seg_lo = 0;
  a.seg_sum = reinterpret_cast<float*>(ws + l.seg_sum);
  a.seg_state = reinterpret_cast<float*>(ws + l.seg_state);
  const bool bf = d->io_dtype == SPARC_BF16;
  if (fwd_wide(l, d->batch, d->modes)) {
    a.n_mb = static_cast<int>((d->modes + 255) / 256);
    if (relu && reset) run_fwd_wide<kRelu | kReset>(a, bf, st);
    else if (relu) run_fwd_wide<kRelu>(a, bf, st);
    else if (reset) run_fwd_wide<kPlanes | kReset>(a, bf, st);
    else run_fwd_wide<kPlanes>(a, bf, st);
  } else if (relu && reset) run_fwd_mode<kRelu | kReset>(a, bf, l.V, st);
  else if (relu) run_fwd_mode<kRelu>(a, bf, l.V, st);
  else if (reset) run_fwd_mode<kPlanes | kReset>(a, bf, l.V, st);
  else run_fwd_mode<kPlanes>(a, bf, l.V, st);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? SPARC_OK : fail(SPARC_EHIP, "p1 fused forward: %s", hipGetErrorString(e));
}

sparc_status p1_fused_backward(const sparc_scan_desc* d, const float* eta, const float* delta,
                               const float* nu_log, const float* theta_log, const void* y_re, const void* y_im,
                               const float* h0_re, const float* h0_im, const int32_t* segment_pos,
                               const void* dy_re, const void* dy_im, const float* dlast_re, const float* dlast_im,
                               void* dw_re, void* dw_im, float* deta, float* ddelta, float* dnu_log,
                               float* dtheta_log, float* dh0_re, float* dh0_im, void* workspace,
                               size_t workspace_bytes, sparc_stream_t stream) {
  if (!p1_fused_shape(d) || d->length <= 0 || (d->flags & SPARC_FLAG_RELU_OUTPUT))
    return fail(SPARC_EINVAL, "p1 fused backward: shape");
  const Layout l = layout(d->batch, d->length, d->modes, 1, true);
  if (workspace_bytes < l.total) return fail(SPARC_EWORKSPACE, "workspace too small: %zu < %zu", workspace_bytes, l.total);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  const int M = static_cast<int>(d->modes);
  float* consts = reinterpret_cast<float*>(ws + l.consts);
  float* part_tok = reinterpret_cast<float*>(ws + l.part_tok);
  float* part_mode = reinterpret_cast<float*>(ws + l.part_mode);
  hipLaunchKernelGGL(mixer_prepare_kernel, dim3(static_cast<unsigned>((M + 255) / 256)), dim3(256), 0, st, M, nu_log,
                     theta_log, nullptr, nullptr, nullptr, consts);
  Args a{};
  a.B = static_cast<int>(d->batch);
  a.T = static_cast<int>(d->length);
  a.M = M;
  a.n_mb = l.n_mb;
  a.consts = consts; a.eta = eta; a.delta = delta;
  a.h_re = const_cast<void*>(y_re); a.h_im = const_cast<void*>(y_im);
  a.dy = dy_re; a.dy_im = dy_im; a.dlast_re = dlast_re; a.dlast_im = dlast_im;
  a.dx = dw_re; a.dw_im = dw_im;
  a.h0_re = h0_re; a.h0_im = h0_im; a.dh0_re = dh0_re; a.dh0_im = dh0_im;
  a.part_tok = part_tok; a.part_mode = part_mode;
  a.n_seg = l.n_seg; a.t_seg = l.t_seg; a.seg_lo = 0;
  a.seg_sum = reinterpret_cast<float*>(ws + l.seg_sum);
  a.seg_state = reinterpret_cast<float*>(ws + l.seg_state);
  a.segpos = segment_pos;
  a.reset_first = (d->flags & SPARC_FLAG_RESET_FIRST) != 0;
  const bool bf = d->io_dtype == SPARC_BF16;
  if (segment_pos || a.reset_first) run_bwd_mode<kPlanes | kReset>(a, bf, l.V, st);
  else run_bwd_mode<kPlanes>(a, bf, l.V, st);
  // d eta, d delta per token over the mode blocks; d nu_log, d theta_log per
  // mode over the (batch row, segment) partial rows
  {
    const float* in[2] = {part_tok, part_tok + static_cast<int64_t>(l.n_mb) * l.R};
    float* out[2] = {deta, ddelta};
    if (sparc_status s = sparc::column_sums(l.n_mb, l.R, 2, in, out, stream)) return s;
  }
  const int64_t prow = d->batch * l.n_seg;
  {
    const float* in[2] = {part_mode, part_mode + prow * d->modes};
    float* out[2] = {dnu_log, dtheta_log};
    if (sparc_status s = sparc::column_sums(prow, d->modes, 2, in, out, stream)) return s;
  }
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? SPARC_OK : fail(SPARC_EHIP, "p1 fused backward: %s", hipGetErrorString(e));
}

}  // namespace sparc

// The controls backward over rows of width W: n_cb column blocks of 2048
// inputs, row blocks of `rows` rows (a multiple of 4 in [16, 128], chosen so
// that the grid has about 1024 workgroups), and the partial direction
// gradients pd [2][n_rb][W] and bias partials pbias [2][n_rb] in the workspace.
struct ControlsLayout {
  int n_cb = 0, n_rb = 0, rows = 0;
  size_t pbias = 0, total = 0;
};

ControlsLayout controls_layout(int64_t R, int64_t W) {
  ControlsLayout c;
  c.n_cb = static_cast<int>((W + 2047) / 2048);
  int64_t rows = (R * c.n_cb + 1023) / 1024;
  rows = (rows + 3) / 4 * 4;
  c.rows = static_cast<int>(rows < 16 ? 16 : (rows > kCtrlBwdRows ? kCtrlBwdRows : rows));
  c.n_rb = static_cast<int>(std::min<int64_t>((R + c.rows - 1) / c.rows, kMaxRowBlocks));
  auto up = [](size_t n) { return (n + 255) / 256 * 256; };
  c.pbias = up(static_cast<size_t>(2) * c.n_rb * W * 4);
  c.total = c.pbias + up(static_cast<size_t>(2) * (c.n_rb > 0 ? c.n_rb : 1) * 4);
  return c;
}

sparc_status check_controls(int64_t rows, int64_t width, int32_t io_dtype) {
  if (io_dtype != SPARC_BF16 && io_dtype != SPARC_F32) return fail(SPARC_EINVAL, "controls: io_dtype must be bf16 or f32");
  if (rows < 0 || rows > (int64_t(1) << 40)) return fail(SPARC_EINVAL, "controls: rows out of range");
  if (width < 8 || width % 8 || width > (int64_t(1) << 30))
    return fail(SPARC_EINVAL, "controls: width must be a positive multiple of 8 (got %lld)", static_cast<long long>(width));
  return SPARC_OK;
}

// The second stream and events of the module backward in time pieces, one set
// per device, created on first use outside graph capture (default priority,
// non-blocking) and kept until the process ends.  The mutex is held while a
// call enqueues its work, so calls from several host threads do not share an
// event between a record and its wait.
struct PipeStreams {
  hipStream_t aux = nullptr;
  hipEvent_t ev[kPieces + 1] = {};
};
std::mutex& pipe_mutex() {
  static std::mutex mu;
  return mu;
}
// The current device's set, or NULL when it does not exist and may not be
// created (create false: the caller's stream is capturing) or when a HIP call
// fails; the error such a failure leaves is cleared, since the caller then
// runs on its own stream alone.  The caller holds pipe_mutex().
PipeStreams* pipe_streams(bool create) {
  static PipeStreams sets[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    return nullptr;
  }
  PipeStreams& ps = sets[dev];
  if (ps.aux) return &ps;
  if (!create) return nullptr;
  for (hipEvent_t& v : ps.ev) {
    if (v) continue;
    if (hipEventCreateWithFlags(&v, hipEventDisableTiming) != hipSuccess) {
      v = nullptr;
      (void)hipGetLastError();
      return nullptr;
    }
  }
  if (hipStreamCreateWithFlags(&ps.aux, hipStreamNonBlocking) != hipSuccess) {
    ps.aux = nullptr;
    (void)hipGetLastError();
    return nullptr;
  }
  return &ps;
}

// Whether st is capturing into a graph (a failed query counts as capturing:
// then nothing is created and nothing waits on the host).
bool stream_capturing(hipStream_t st) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess) {
    (void)hipGetLastError();
    return true;
  }
  return cs != hipStreamCaptureStatusNone;
}

// The module backward in l.n_seg time pieces, the last first.  On the caller's
// stream: the mixer backward of piece p (entering adjoint from piece p + 1),
// then the sums of its per-token partials into d eta, d delta of its rows; on
// the second stream, after an event: the controls backward of piece p (dx of
// its rows in place, the direction partials of its row blocks), which so runs
// beside the mixer backward of piece p - 1.  The caller's stream waits for
// the second stream before the per-mode and direction sums, and before any
// error return once the second stream has been forked.  Without the second
// stream (a capture that reaches the first call, a failed stream or event
// call) every launch goes to the caller's stream, in the same order and with
// the same workspace layout.
sparc_status piped_backward(const Layout& l, int64_t batch, int64_t length, int64_t modes, int32_t io_dtype,
                            const void* x, const float* phase_direction, const float* radial_direction,
                            const float* eta, const float* delta, const float* nu_log, const float* theta_log,
                            const float* write_log_gain, const float* write_phase_response,
                            const float* write_radial_response, const void* h_re, const void* h_im, const void* dy,
                            const float* dlast_re, const float* dlast_im, void* dx, float* dphase_direction,
                            float* dradial_direction, float* dnu_log, float* dtheta_log, float* dwrite_log_gain,
                            float* dwrite_phase_response, float* dwrite_radial_response, char* ws, hipStream_t st) {
  std::lock_guard<std::mutex> lock(pipe_mutex());
  const bool capturing = stream_capturing(st);
  PipeStreams* ps = pipe_streams(!capturing);
  const sparc_stream_t stream = reinterpret_cast<sparc_stream_t>(st);
  const int M = static_cast<int>(modes), W = 2 * M;
  float* consts = reinterpret_cast<float*>(ws + l.consts);
  float* part_tok = reinterpret_cast<float*>(ws + l.part_tok);
  float* part_mode = reinterpret_cast<float*>(ws + l.part_mode);
  float* deta = reinterpret_cast<float*>(ws + l.tok);
  float* ddelta = deta + l.R;
  float* pd = reinterpret_cast<float*>(ws + l.pd);
  float* pbias = reinterpret_cast<float*>(ws + l.pbias);
  Args a{};
  a.B = static_cast<int>(batch);
  a.T = static_cast<int>(length);
  a.M = M;
  a.n_mb = l.n_mb;
  a.x = x; a.consts = consts; a.eta = eta; a.delta = delta;
  a.h_re = const_cast<void*>(h_re); a.h_im = const_cast<void*>(h_im);
  a.dy = dy; a.dlast_re = dlast_re; a.dlast_im = dlast_im; a.dx = dx;
  a.part_tok = part_tok; a.part_mode = part_mode;
  a.n_seg = l.n_seg; a.t_seg = l.t_seg;
  a.seg_state = reinterpret_cast<float*>(ws + l.seg_state);
  a.piped = 1;
  const int64_t L = l.t_seg, rows_p = batch * L;
  const dim3 gb(static_cast<unsigned>((W + 2047) / 2048), static_cast<unsigned>(l.n_rb_piece));
  // the controls go to the second stream while every event call succeeds,
  // else (from then on) to the caller's stream, in order after the mixer
  hipEvent_t fork = ps ? ps->ev[kPieces] : nullptr;
  bool forked = false;  // the second stream waits on the fork and must be joined
  if (ps) {
    if (hipEventRecord(fork, st) == hipSuccess && hipStreamWaitEvent(ps->aux, fork, 0) == hipSuccess) forked = true;
    else (void)hipGetLastError();
  }
  hipStream_t cs = forked ? ps->aux : st;
  hipLaunchKernelGGL(mixer_prepare_kernel, dim3(static_cast<unsigned>((M + 255) / 256)), dim3(256), 0, st, M, nu_log,
                     theta_log, write_log_gain, write_phase_response, write_radial_response, consts);
  // the caller's stream waits for everything enqueued on the second stream;
  // if that cannot be enqueued, the host waits for the second stream (never
  // while capturing: a capture with an unjoined stream fails at its end)
  auto join = [&]() -> hipError_t {
    if (!forked) return hipSuccess;
    forked = false;
    cs = st;
    hipError_t e = hipEventRecord(fork, ps->aux);
    if (e == hipSuccess) e = hipStreamWaitEvent(st, fork, 0);
    if (e != hipSuccess && !capturing) (void)hipStreamSynchronize(ps->aux);
    return e;
  };
  for (int p = l.n_seg - 1; p >= 0; --p) {
    a.seg_lo = p;
    if (io_dtype == SPARC_BF16) launch_bwd<sparc::bf16, 1, false, kModule>(a, 1, st);
    else launch_bwd<float, 1, false, kModule>(a, 1, st);
    const float* pt = part_tok + static_cast<int64_t>(p) * 2 * l.n_mb * rows_p;
    float* de = deta + static_cast<int64_t>(p) * rows_p;
    float* dd = ddelta + static_cast<int64_t>(p) * rows_p;
    const float* in[2] = {pt, pt + static_cast<int64_t>(l.n_mb) * rows_p};
    float* out[2] = {de, dd};
    sparc_status s = sparc::column_sums(l.n_mb, rows_p, 2, in, out, stream);
    if (s) {
      (void)join();
      return s;
    }
    if (cs != st && (hipEventRecord(ps->ev[p], st) != hipSuccess || hipStreamWaitEvent(cs, ps->ev[p], 0) != hipSuccess)) {
      (void)hipGetLastError();
      cs = st;  // the second stream stays forked until the join
    }
    const int64_t t0 = static_cast<int64_t>(p) * L;
    const int rb0 = p * l.n_rb_piece;
    if (io_dtype == SPARC_BF16)
      hipLaunchKernelGGL(ctrl_bwd_kernel<sparc::bf16>, gb, dim3(256), 0, cs, rows_p, W, kCtrlBwdRows, x,
                         phase_direction, radial_direction, eta, delta, de, dd, dx, pd, pbias, length, t0, L, rb0,
                         l.n_rb);
    else
      hipLaunchKernelGGL(ctrl_bwd_kernel<float>, gb, dim3(256), 0, cs, rows_p, W, kCtrlBwdRows, x,
                         phase_direction, radial_direction, eta, delta, de, dd, dx, pd, pbias, length, t0, L, rb0,
                         l.n_rb);
    if (hipError_t le = hipGetLastError()) {
      (void)join();
      return fail(SPARC_EHIP, "mixer backward: controls launch: %s", hipGetErrorString(le));
    }
  }
  hipError_t e = join();
  if (e != hipSuccess) return fail(SPARC_EHIP, "mixer backward: stream join: %s", hipGetErrorString(e));
  float* outs[5] = {dnu_log, dtheta_log, dwrite_log_gain, dwrite_phase_response, dwrite_radial_response};
  const int64_t prow = batch * l.n_seg;  // one partial row per (batch row, piece)
  {
    const float* in[5];
    for (int p = 0; p < 5; ++p) in[p] = part_mode + static_cast<int64_t>(p) * prow * modes;
    if (sparc_status s = sparc::column_sums(prow, modes, 5, in, outs, stream)) return s;
  }
  if (sparc_status s = direction_sums(l.n_rb, W, pd, pbias, dphase_direction, dradial_direction, stream)) return s;
  e = hipGetLastError();
  return e == hipSuccess ? SPARC_OK : fail(SPARC_EHIP, "mixer backward: %s", hipGetErrorString(e));
}

// ---------------------------------------------------------------------------
// the module backward in one launch (kCoop)
// ---------------------------------------------------------------------------
// Which form sparc_mixer_backward takes: 0 the one-launch form wherever it
// fits (below), 1 never (time pieces or the separate controls backward).
std::atomic<int> g_bwd_plan{0};

// Steps per block of the one-launch form: 4 (with 8 the ring and the
// reduction's registers spill under the two-waves-per-SIMD bound).
constexpr int kCoopS = 4;
template <typename IO, int kS>
const void* coop_kernel() {
  return reinterpret_cast<const void*>(&mixer_bwd_kernel<IO, 1, kS, false, kModule | kCoop>);
}
// Workgroups of the kernel that the current device holds at once (0 on any
// failure), cached per device.
template <typename IO, int kS>
int64_t coop_capacity() {
  static std::atomic<int64_t> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    return 0;
  }
  int64_t c = cache[dev].load(std::memory_order_relaxed);
  if (c > 0) return c;
  int per_cu = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, coop_kernel<IO, kS>(), 64, 0) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  c = static_cast<int64_t>(per_cu) * cus;
  cache[dev].store(c, std::memory_order_relaxed);
  return c;
}

struct CoopLayout {
  int kS = 0, nblk = 0, n_mb = 0;
  size_t consts = 0, part_mode = 0, part = 0, sum = 0, dtok = 0, pd = 0, total = 0;
};
// Byte 4 of the workspace is the error word (as for the scans, so that
// sparc_scan_workspace_error reads it).
CoopLayout coop_layout(int64_t B, int64_t T, int64_t M, int kS) {
  CoopLayout c;
  c.kS = kS;
  c.n_mb = static_cast<int>((M + 63) / 64);
  c.nblk = static_cast<int>((T + kS - 1) / kS);
  auto up = [](size_t n) { return (n + 255) / 256 * 256; };
  size_t off = 256;
  c.consts = off;
  off += up(static_cast<size_t>(M) * kConsts * 4);
  c.part_mode = off;
  off += up(static_cast<size_t>(5) * B * M * 4);
  c.part = off;
  off += up(static_cast<size_t>(B) * c.nblk * c.n_mb * 2 * kS * 4);
  c.sum = off;
  off += up(static_cast<size_t>(B) * c.nblk * 2 * kS * 4);
  c.dtok = off;
  off += up(static_cast<size_t>(2) * B * T * 4);
  c.pd = off;
  off += up(static_cast<size_t>(2) * B * 2 * M * 4);
  c.total = off;
  return c;
}

// The steps per block of the one-launch form for this call, or 0 where it
// does not apply: the plan allows it, T > 0, one mode per lane and no time
// segments (the chains fill the GPU), and every chain resident at once.
int coop_steps(int64_t B, int64_t T, int64_t M, int32_t io) {
  if (g_bwd_plan.load(std::memory_order_relaxed) != 0 || T <= 0) return 0;
  const Layout l = layout(B, T, M, 1);
  if (l.V != 1 || l.n_seg != 1) return 0;
  const int64_t grid = B * l.n_mb;
  const int64_t cap = io == SPARC_BF16 ? coop_capacity<sparc::bf16, kCoopS>() : coop_capacity<float, kCoopS>();
  return grid <= cap ? kCoopS : 0;
}

sparc_status coop_backward(int kS, int64_t batch, int64_t length, int64_t modes, int32_t io_dtype, const void* x,
                           const float* phase_direction, const float* radial_direction, const float* eta,
                           const float* delta, const float* nu_log, const float* theta_log,
                           const float* write_log_gain, const float* write_phase_response,
                           const float* write_radial_response, const void* h_re, const void* h_im, const void* dy,
                           const float* dlast_re, const float* dlast_im, void* dx, float* dphase_direction,
                           float* dradial_direction, float* dnu_log, float* dtheta_log, float* dwrite_log_gain,
                           float* dwrite_phase_response, float* dwrite_radial_response, char* ws, hipStream_t st) {
  const CoopLayout c = coop_layout(batch, length, modes, kS);
  const sparc_stream_t stream = reinterpret_cast<sparc_stream_t>(st);
  const int M = static_cast<int>(modes), W = 2 * M;
  float* consts = reinterpret_cast<float*>(ws + c.consts);
  hipLaunchKernelGGL(mixer_prepare_kernel, dim3(static_cast<unsigned>((M + 255) / 256)), dim3(256), 0, st, M, nu_log,
                     theta_log, write_log_gain, write_phase_response, write_radial_response, consts);
  // the error word starts at zero, the records and the blocks' gradients as
  // kCoopEmpty (fill kernels, not memsets: the call may be captured into a
  // graph; the records and gradients are adjacent)
  // (one launch of 16-byte stores: the offsets are multiples of 256 bytes)
  const int64_t nfill4 = static_cast<int64_t>(c.dtok - c.part) / 16;
  hipLaunchKernelGGL(fill_u32x4_kernel, dim3(static_cast<unsigned>((nfill4 + 255) / 256)), dim3(256), 0, st,
                     reinterpret_cast<uint4*>(ws + c.part), nfill4, kCoopEmpty, reinterpret_cast<uint32_t*>(ws), 2, 0u);
  Args a{};
  a.B = static_cast<int>(batch);
  a.T = static_cast<int>(length);
  a.M = M;
  a.n_mb = c.n_mb;
  a.x = x; a.consts = consts; a.eta = eta; a.delta = delta;
  a.h_re = const_cast<void*>(h_re); a.h_im = const_cast<void*>(h_im);
  a.dy = dy; a.dlast_re = dlast_re; a.dlast_im = dlast_im; a.dx = dx;
  a.part_mode = reinterpret_cast<float*>(ws + c.part_mode);
  a.n_seg = 1; a.t_seg = static_cast<int>(length); a.seg_lo = 0;
  a.pdir = phase_direction;
  a.rdir = radial_direction;
  a.coop_part = reinterpret_cast<float*>(ws + c.part);
  a.coop_sum = reinterpret_cast<float*>(ws + c.sum);
  a.coop_dtok = reinterpret_cast<float*>(ws + c.dtok);
  a.coop_pd = reinterpret_cast<float*>(ws + c.pd);
  a.coop_nblk = c.nblk;
  a.coop_error = reinterpret_cast<uint32_t*>(ws) + 1;
  a.coop_spin = sparc::wait_limit();
  const dim3 g(static_cast<unsigned>(batch * c.n_mb));
  constexpr int kC = kModule | kCoop;
  static_assert(kCoopS == 4, "one instantiation per I/O type");
  if (kS != kCoopS) return fail(SPARC_EINVAL, "mixer backward: steps per block");
  if (io_dtype == SPARC_BF16)
    hipLaunchKernelGGL((mixer_bwd_kernel<sparc::bf16, 1, kCoopS, false, kC>), g, dim3(64), 0, st, a);
  else
    hipLaunchKernelGGL((mixer_bwd_kernel<float, 1, kCoopS, false, kC>), g, dim3(64), 0, st, a);
  if (hipError_t le = hipGetLastError()) return fail(SPARC_EHIP, "mixer backward: %s", hipGetErrorString(le));
  float* outs[5] = {dnu_log, dtheta_log, dwrite_log_gain, dwrite_phase_response, dwrite_radial_response};
  {
    const float* in[5];
    for (int p = 0; p < 5; ++p) in[p] = a.part_mode + static_cast<int64_t>(p) * batch * modes;
    if (sparc_status s = sparc::column_sums(batch, modes, 5, in, outs, stream)) return s;
  }
  const int64_t R = batch * length;
  {
    const float* in[2] = {a.coop_pd, a.coop_pd + batch * W};
    float* out[2] = {dphase_direction, dradial_direction};
    if (sparc_status s = sparc::column_sums(batch, W, 2, in, out, stream)) return s;
  }
  {
    const float* in[2] = {a.coop_dtok, a.coop_dtok + R};
    float* out[2] = {dphase_direction + W, dradial_direction + W};
    if (sparc_status s = sparc::column_sums(R, 1, 2, in, out, stream)) return s;
  }
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? SPARC_OK : fail(SPARC_EHIP, "mixer backward: %s", hipGetErrorString(e));
}

extern "C" {

size_t sparc_mixer_workspace_bytes(int64_t batch, int64_t length, int64_t modes, int direction) {
  if (batch <= 0 || length < 0 || modes <= 0 || modes % 4 || (direction != 0 && direction != 1)) return 0;
  // the module backward may run in time pieces or in one launch (larger workspaces)
  size_t n = std::max(layout(batch, length, modes, direction).total, layout(batch, length, modes, direction, false, true).total);
  if (direction == 1) n = std::max(n, coop_layout(batch, length, modes, kCoopS).total);
  return n;
}

int sparc_mixer_backward_plan(int plan) {
  if (plan != 0 && plan != 1) return -1;
  return g_bwd_plan.exchange(plan, std::memory_order_relaxed);
}

int sparc_mixer_backward_form(int64_t batch, int64_t length, int64_t modes, int32_t io_dtype) {
  if (check_shape(batch, length, modes, io_dtype)) return -1;
  if (coop_steps(batch, length, modes, io_dtype)) return 2;
  return layout(batch, length, modes, 1, false, true).piped ? 1 : 0;
}

sparc_status sparc_mixer_scan_forward(int64_t batch, int64_t length, int64_t modes, int32_t io_dtype,
                                      const void* x, const float* eta, const float* delta, const float* nu_log,
                                      const float* theta_log, const float* write_log_gain,
                                      const float* write_phase_response, const float* write_radial_response,
                                      void* y, void* h_re, void* h_im, float* last_re, float* last_im,
                                      void* workspace, size_t workspace_bytes, sparc_stream_t stream) {
  if (sparc_status s = check_shape(batch, length, modes, io_dtype)) return s;
  // per-token tensors may be NULL when length is 0 (nothing is read or written)
  const bool rows = length > 0;
  if ((rows && (!x || !eta || !delta || !y || !h_re || !h_im)) ||
      !params_ok(nu_log, theta_log, write_log_gain, write_phase_response, write_radial_response))
    return fail(SPARC_EINVAL, "mixer scan forward: NULL pointer");
  if ((last_re == nullptr) != (last_im == nullptr)) return fail(SPARC_EINVAL, "mixer scan forward: last_re/last_im");
  const Layout l = layout(batch, length, modes, 0);
  if (!workspace || workspace_bytes < l.total)
    return fail(SPARC_EWORKSPACE, "mixer scan forward: workspace too small (%zu < %zu)", workspace_bytes, l.total);
  const size_t esz = io_dtype == SPARC_BF16 ? 2 : 4;
  if (!al(x, 16) || !al(y, 16) || !al(h_re, esz * l.V) || !al(h_im, esz * l.V) || !al(workspace, 256))
    return fail(SPARC_EINVAL, "mixer scan forward: misaligned tensor");
  return scan_forward_impl(l, batch, length, modes, io_dtype, x, eta, delta, nu_log, theta_log, write_log_gain,
                           write_phase_response, write_radial_response, y, h_re, h_im, last_re, last_im,
                           static_cast<char*>(workspace), reinterpret_cast<hipStream_t>(stream));
}

sparc_status sparc_mixer_forward(int64_t batch, int64_t length, int64_t modes, int32_t io_dtype,
                                 const void* x, const float* phase_direction, const float* radial_direction,
                                 const float* nu_log, const float* theta_log, const float* write_log_gain,
                                 const float* write_phase_response, const float* write_radial_response,
                                 float* eta, float* delta, void* y, void* h_re, void* h_im,
                                 float* last_re, float* last_im, void* workspace, size_t workspace_bytes,
                                 sparc_stream_t stream) {
  if (sparc_status s = check_shape(batch, length, modes, io_dtype)) return s;
  const bool rows = length > 0;  // per-token tensors may be NULL when length is 0
  if ((rows && (!x || !eta || !delta || !y || !h_re || !h_im)) || !phase_direction || !radial_direction ||
      !params_ok(nu_log, theta_log, write_log_gain, write_phase_response, write_radial_response))
    return fail(SPARC_EINVAL, "mixer forward: NULL pointer");
  if ((last_re == nullptr) != (last_im == nullptr)) return fail(SPARC_EINVAL, "mixer forward: last_re/last_im");
  const Layout l = layout(batch, length, modes, 0);
  if (!workspace || workspace_bytes < l.total)
    return fail(SPARC_EWORKSPACE, "mixer forward: workspace too small (%zu < %zu)", workspace_bytes, l.total);
  const size_t esz = io_dtype == SPARC_BF16 ? 2 : 4;
  if (!al(x, 16) || !al(y, 16) || !al(h_re, esz * l.V) || !al(h_im, esz * l.V) || !al(phase_direction, 16) ||
      !al(radial_direction, 16) || !al(workspace, 256))
    return fail(SPARC_EINVAL, "mixer forward: misaligned tensor");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int W = 2 * static_cast<int>(modes);
  if (length > 0) {
    if (io_dtype == SPARC_BF16)
      launch_ctrl_fwd<sparc::bf16>(st, l.R, W, x, phase_direction, radial_direction, eta, delta);
    else
      launch_ctrl_fwd<float>(st, l.R, W, x, phase_direction, radial_direction, eta, delta);
  }
  return scan_forward_impl(l, batch, length, modes, io_dtype, x, eta, delta, nu_log, theta_log, write_log_gain,
                           write_phase_response, write_radial_response, y, h_re, h_im, last_re, last_im,
                           static_cast<char*>(workspace), st);
}

sparc_status sparc_mixer_scan_backward(int64_t batch, int64_t length, int64_t modes, int32_t io_dtype,
                                       const void* x, const float* eta, const float* delta, const float* nu_log,
                                       const float* theta_log, const float* write_log_gain,
                                       const float* write_phase_response, const float* write_radial_response,
                                       const void* h_re, const void* h_im, const void* dy, const float* dlast_re,
                                       const float* dlast_im, void* dx, float* deta, float* ddelta, float* dnu_log,
                                       float* dtheta_log, float* dwrite_log_gain, float* dwrite_phase_response,
                                       float* dwrite_radial_response, void* workspace, size_t workspace_bytes,
                                       sparc_stream_t stream) {
  if (sparc_status s = check_shape(batch, length, modes, io_dtype)) return s;
  const bool rows = length > 0;  // per-token tensors may be NULL when length is 0
  if ((rows && (!x || !eta || !delta || !h_re || !h_im || !dy || !dx || !deta || !ddelta)) ||
      !params_ok(nu_log, theta_log, write_log_gain, write_phase_response, write_radial_response) ||
      !params_ok(dnu_log, dtheta_log, dwrite_log_gain, dwrite_phase_response, dwrite_radial_response))
    return fail(SPARC_EINVAL, "mixer scan backward: NULL pointer");
  if ((dlast_re == nullptr) != (dlast_im == nullptr)) return fail(SPARC_EINVAL, "mixer scan backward: dlast_re/dlast_im");
  const Layout l = layout(batch, length, modes, 1);
  if (!workspace || workspace_bytes < l.total)
    return fail(SPARC_EWORKSPACE, "mixer scan backward: workspace too small (%zu < %zu)", workspace_bytes, l.total);
  const size_t esz = io_dtype == SPARC_BF16 ? 2 : 4;
  if (!al(x, 16) || !al(dy, 16) || !al(dx, 16) || !al(h_re, esz * l.V) || !al(h_im, esz * l.V) || !al(workspace, 256))
    return fail(SPARC_EINVAL, "mixer scan backward: misaligned tensor");
  return scan_backward_impl(l, batch, length, modes, io_dtype, x, eta, delta, nu_log, theta_log, write_log_gain,
                            write_phase_response, write_radial_response, h_re, h_im, dy, dlast_re, dlast_im, dx,
                            deta, ddelta, dnu_log, dtheta_log, dwrite_log_gain, dwrite_phase_response,
                            dwrite_radial_response, static_cast<char*>(workspace), stream);
}

sparc_status sparc_mixer_backward(int64_t batch, int64_t length, int64_t modes, int32_t io_dtype,
                                  const void* x, const float* phase_direction, const float* radial_direction,
                                  const float* nu_log, const float* theta_log, const float* write_log_gain,
                                  const float* write_phase_response, const float* write_radial_response,
                                  const float* eta, const float* delta, const void* h_re, const void* h_im,
                                  const void* dy, const float* dlast_re, const float* dlast_im, void* dx,
                                  float* dphase_direction, float* dradial_direction, float* dnu_log,
                                  float* dtheta_log, float* dwrite_log_gain, float* dwrite_phase_response,
                                  float* dwrite_radial_response, void* workspace, size_t workspace_bytes,
                                  sparc_stream_t stream) {
  if (sparc_status s = check_shape(batch, length, modes, io_dtype)) return s;
  const bool rows = length > 0;  // per-token tensors may be NULL when length is 0
  if ((rows && (!x || !eta || !delta || !h_re || !h_im || !dy || !dx)) || !phase_direction ||
      !radial_direction || !dphase_direction || !dradial_direction ||
      !params_ok(nu_log, theta_log, write_log_gain, write_phase_response, write_radial_response) ||
      !params_ok(dnu_log, dtheta_log, dwrite_log_gain, dwrite_phase_response, dwrite_radial_response))
    return fail(SPARC_EINVAL, "mixer backward: NULL pointer");
  if ((dlast_re == nullptr) != (dlast_im == nullptr)) return fail(SPARC_EINVAL, "mixer backward: dlast_re/dlast_im");
  const Layout l = layout(batch, length, modes, 1, false, true);
  const int cs = coop_steps(batch, length, modes, io_dtype);
  const size_t need = cs ? coop_layout(batch, length, modes, cs).total : l.total;
  if (!workspace || workspace_bytes < need)
    return fail(SPARC_EWORKSPACE, "mixer backward: workspace too small (%zu < %zu)", workspace_bytes, need);
  const size_t esz = io_dtype == SPARC_BF16 ? 2 : 4;
  if (!al(x, 16) || !al(dy, 16) || !al(dx, 16) || !al(h_re, esz * l.V) || !al(h_im, esz * l.V) ||
      !al(phase_direction, 16) || !al(radial_direction, 16) || !al(workspace, 256))
    return fail(SPARC_EINVAL, "mixer backward: misaligned tensor");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int M = static_cast<int>(modes), W = 2 * M;
  char* ws = static_cast<char*>(workspace);
  if (cs)
    return coop_backward(cs, batch, length, modes, io_dtype, x, phase_direction, radial_direction, eta, delta, nu_log,
                         theta_log, write_log_gain, write_phase_response, write_radial_response, h_re, h_im, dy,
                         dlast_re, dlast_im, dx, dphase_direction, dradial_direction, dnu_log, dtheta_log,
                         dwrite_log_gain, dwrite_phase_response, dwrite_radial_response, ws, st);
  float* deta = reinterpret_cast<float*>(ws + l.tok);
  float* ddelta = deta + l.R;
  if (l.piped)
    return piped_backward(l, batch, length, modes, io_dtype, x, phase_direction, radial_direction, eta, delta,
                          nu_log, theta_log, write_log_gain, write_phase_response, write_radial_response, h_re, h_im,
                          dy, dlast_re, dlast_im, dx, dphase_direction, dradial_direction, dnu_log, dtheta_log,
                          dwrite_log_gain, dwrite_phase_response, dwrite_radial_response, ws, st);
  if (sparc_status s = scan_backward_impl(l, batch, length, modes, io_dtype, x, eta, delta, nu_log, theta_log,
                                          write_log_gain, write_phase_response, write_radial_response, h_re, h_im,
                                          dy, dlast_re, dlast_im, dx, deta, ddelta, dnu_log, dtheta_log,
                                          dwrite_log_gain, dwrite_phase_response, dwrite_radial_response, ws, stream))
    return s;
  if (length == 0) {
    const dim3 gz(static_cast<unsigned>((W + 1 + 255) / 256));
    for (float* o : {dphase_direction, dradial_direction})
      hipLaunchKernelGGL(fill_zero_f32_kernel, gz, dim3(256), 0, st, o, static_cast<int64_t>(W + 1));
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? SPARC_OK : fail(SPARC_EHIP, "mixer backward: %s", hipGetErrorString(e));
  }
  float* pd = reinterpret_cast<float*>(ws + l.pd);
  float* pbias = reinterpret_cast<float*>(ws + l.pbias);
  const dim3 gb(static_cast<unsigned>((W + 2047) / 2048), static_cast<unsigned>(l.n_rb));
  if (io_dtype == SPARC_BF16)
    hipLaunchKernelGGL(ctrl_bwd_kernel<sparc::bf16>, gb, dim3(256), 0, st, l.R, W, kCtrlBwdRows, x, phase_direction,
                       radial_direction, eta, delta, deta, ddelta, dx, pd, pbias, l.R, int64_t(0), l.R, 0, l.n_rb);
  else
    hipLaunchKernelGGL(ctrl_bwd_kernel<float>, gb, dim3(256), 0, st, l.R, W, kCtrlBwdRows, x, phase_direction,
                       radial_direction, eta, delta, deta, ddelta, dx, pd, pbias, l.R, int64_t(0), l.R, 0, l.n_rb);
  // direction gradients: columns 0..W-1 from the row-block partials, the bias from pbias
  if (sparc_status s = direction_sums(l.n_rb, W, pd, pbias, dphase_direction, dradial_direction, stream)) return s;
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? SPARC_OK : fail(SPARC_EHIP, "mixer backward: %s", hipGetErrorString(e));
}

// ---------------------------------------------------------------------------
// the controls alone, over rows of any width that is a multiple of 8
// ---------------------------------------------------------------------------
size_t sparc_controls_workspace_bytes(int64_t rows, int64_t width) {
  if (rows < 0 || width < 8 || width % 8 || width > (int64_t(1) << 30)) return 0;
  const ControlsLayout c = controls_layout(rows, width);
  return c.total;
}

sparc_status sparc_controls_forward(int64_t rows, int64_t width, int32_t io_dtype, const void* x,
                                    const float* phase_direction, const float* radial_direction, float* eta,
                                    float* delta, sparc_stream_t stream) {
  if (sparc_status s = check_controls(rows, width, io_dtype)) return s;
  if (rows == 0) return SPARC_OK;  // nothing to read or write (the pointers may be NULL)
  if (!x || !phase_direction || !radial_direction || !eta || !delta)
    return fail(SPARC_EINVAL, "controls forward: NULL pointer");
  if (!al(x, 16) || !al(phase_direction, 16) || !al(radial_direction, 16))
    return fail(SPARC_EINVAL, "controls forward: misaligned tensor");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int W = static_cast<int>(width);
  if (io_dtype == SPARC_BF16)
    launch_ctrl_fwd<sparc::bf16>(st, rows, W, x, phase_direction, radial_direction, eta, delta);
  else
    launch_ctrl_fwd<float>(st, rows, W, x, phase_direction, radial_direction, eta, delta);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? SPARC_OK : fail(SPARC_EHIP, "controls forward: %s", hipGetErrorString(e));
}

sparc_status sparc_controls_backward(int64_t rows, int64_t width, int32_t io_dtype, const void* x,
                                     const float* phase_direction, const float* radial_direction, const float* eta,
                                     const float* delta, const float* deta, const float* ddelta, void* dx,
                                     float* dphase_direction, float* dradial_direction, void* workspace,
                                     size_t workspace_bytes, sparc_stream_t stream) {
  if (sparc_status s = check_controls(rows, width, io_dtype)) return s;
  if (!dphase_direction || !dradial_direction) return fail(SPARC_EINVAL, "controls backward: NULL pointer");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int W = static_cast<int>(width);
  if (rows == 0) {  // zero direction gradients; the row tensors may be NULL
    const dim3 gz(static_cast<unsigned>((W + 1 + 255) / 256));
    for (float* o : {dphase_direction, dradial_direction})
      hipLaunchKernelGGL(fill_zero_f32_kernel, gz, dim3(256), 0, st, o, static_cast<int64_t>(W + 1));
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? SPARC_OK : fail(SPARC_EHIP, "controls backward: %s", hipGetErrorString(e));
  }
  if (!x || !phase_direction || !radial_direction || !eta || !delta || !deta || !ddelta || !dx)
    return fail(SPARC_EINVAL, "controls backward: NULL pointer");
  const ControlsLayout c = controls_layout(rows, width);
  if (!workspace || workspace_bytes < c.total)
    return fail(SPARC_EWORKSPACE, "controls backward: workspace too small (%zu < %zu)", workspace_bytes, c.total);
  if (!al(x, 16) || !al(dx, 16) || !al(phase_direction, 16) || !al(radial_direction, 16) || !al(workspace, 256))
    return fail(SPARC_EINVAL, "controls backward: misaligned tensor");
  char* ws = static_cast<char*>(workspace);
  float* pd = reinterpret_cast<float*>(ws);
  float* pbias = reinterpret_cast<float*>(ws + c.pbias);
  const dim3 gb(static_cast<unsigned>(c.n_cb), static_cast<unsigned>(c.n_rb));
  if (io_dtype == SPARC_BF16)
    hipLaunchKernelGGL(ctrl_bwd_kernel<sparc::bf16>, gb, dim3(256), 0, st, rows, W, c.rows, x, phase_direction,
                       radial_direction, eta, delta, deta, ddelta, dx, pd, pbias, rows, int64_t(0), rows, 0, c.n_rb);
  else
    hipLaunchKernelGGL(ctrl_bwd_kernel<float>, gb, dim3(256), 0, st, rows, W, c.rows, x, phase_direction,
                       radial_direction, eta, delta, deta, ddelta, dx, pd, pbias, rows, int64_t(0), rows, 0, c.n_rb);
  if (sparc_status s = direction_sums(c.n_rb, W, pd, pbias, dphase_direction, dradial_direction, stream)) return s;
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? SPARC_OK : fail(SPARC_EHIP, "controls backward: %s", hipGetErrorString(e));
}

}  // extern "C"
