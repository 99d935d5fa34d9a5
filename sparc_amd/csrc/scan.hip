// SPARC chunked diagonal linear scan for gfx950: forward and backward.
//
// h_t = a_t * h_{t-1} + w_t over T steps for every (batch row, mode), complex
// (M modes, planar re/im tensors) or real, fp32 state, bf16 or fp32 I/O.
//
// Work decomposition (both directions)
//   tile  = (batch row b, mode block of 64*V modes, chunk of C = S*NW steps)
//   chain = the tiles of one (b, mode block), ordered in time
//   one workgroup = NW waves per tile; wave k owns steps [k*S, (k+1)*S) of the
//   chunk and every lane owns V adjacent modes, so each step of a wave is one
//   coalesced V-element load per plane.
// Single pass: every input element is loaded from HBM once, kept in
// registers, summarised, and replayed once the carry into the chunk is known.
//   1. each wave scans its S steps from a zero state -> (P_k, Q_k), the affine
//      map "state in -> state out" of its sub-chunk (P = prod a, Q = local h);
//   2. the NW maps are composed in LDS into the tile aggregate;
//   3. the tile publishes its aggregate, then looks back along its chain
//      (decoupled look-back) until it finds a published inclusive carry,
//      composing aggregates on the way; it publishes its own inclusive carry
//      (= the state after its last step, which is also the saved chunk state
//      the backward recomputes from);
//   4. every wave replays its S steps from its exact start state and stores.
// Tiles are claimed through an atomic ticket in chunk-major order, so every
// tile's predecessors were claimed earlier by running workgroups: the
// look-back waits always end.  The waits are bounded anyway (lb_window).
//
// The backward runs the same machinery on the adjoint in reverse time
// (lambda_{t-1} = conj(a_t) lambda_t + dy_{t-1}) after recomputing the
// forward states of the chunk from the saved chunk state, so no [B,T,M]
// state is stored by the forward.
//
// Reference kernels replaced: _sparc_chunk_summary / _sparc_chunk_prefix /
// _sparc_chunk_replay (sparc-kernal/forward/scan.py:885-1003, 1276-1354),
// the hierarchical and grouped carries (forward/scan.py:1082-1273), the real
// and complex scans (forward/scan.py:621-722), the serial SPARC scans
// (forward/scan.py:724-854) and their reverse-time counterparts
// (sparc-kernal/backward/scan.py:34-781).

#include <atomic>
#include <type_traits>

#include "common.h"
#include "p1_fused.h"
#include "reduce.h"
#include "sparc_hip.h"

// SPARC_SCAN_PART: which part of a split build this is (see the host side)
#ifndef SPARC_SCAN_PART
#define SPARC_SCAN_PART -1
#endif
#define SPARC_SCAN_OWNS(k) (SPARC_SCAN_PART < 0 || SPARC_SCAN_PART == (k))

namespace sparc {


// How a lane's V modes map to gates.
enum GateMode : int {
  GATE_LANE = 0,   // all V modes of a lane share one gate; a group fits in one tile
  GATE_MODE = 1,   // one gate per mode (G == M)
  GATE_CROSS = 2   // group spans several tiles (or G == 1): partial sums per tile
};

struct ScanArgs {
  int B, T, M, G, gs;
  int n_chunks, n_mblocks, n_chains;
  uint32_t flags;
  uint32_t spin_limit;
  const void* g0;
  const void* g1;
  const float* nu_log;
  const float* theta_log;
  const void* w_re;
  const void* w_im;
  const float* h0_re;
  const float* h0_im;
  const int32_t* segpos;
  void* y_re;
  void* y_im;
  float* chunk_state;
  // backward
  const float* chunk_state_in;
  const void* dy_re;
  const void* dy_im;
  const float* dlast_re;
  const float* dlast_im;
  void* dw_re;
  void* dw_im;
  void* dg0;
  void* dg1;
  float* part_g0;     // [B*T, n_mblocks] (GATE_CROSS)
  float* part_g1;
  float* part_nu;     // [B*n_chunks, M] (P1)
  float* part_theta;
  float* dh0_re;
  float* dh0_im;
  // workspace
  uint32_t* ticket;
  uint32_t* error;
  uint32_t* flagv;    // [n_chains, n_chunks]
  float* agg;         // [n_chains, n_chunks, 64*V, NQ]
  float* carry;       // backward inclusive adjoint carries [B, n_chunks, M, NH]
  // time segments of the serial kernels (n_seg > 1): a launch runs segments
  // seg_lo, seg_lo + 1, ... of t_seg steps each (grid = n_chains * segments)
  int n_seg, t_seg, seg_lo;
  float* seg_sum;     // [B][n_seg][M][4]: each segment's map (P, Q) of the state or adjoint
  float* seg_state;   // [B][n_seg][M][2]: the state (forward) or adjoint (backward) entering it
};

// Cache policy of the serial kernels' plane loads and stores: bit 0 loads,
// bit 1 stores non-temporal (forward and backward separately).
#ifndef SPARC_FWD_NT
#define SPARC_FWD_NT 3
#endif
#ifndef SPARC_BWD_NT
#define SPARC_BWD_NT 3
#endif
// Cache policy of the look-back kernels' streamed planes (w, y, dy, dw): bit 0
// non-temporal loads, bit 1 non-temporal stores.  Measured at B=4, T=65536,
// M=4096 (real, fp32): both non-temporal 1.64 / 2.66 ms forward / backward,
// neither 1.72 / 2.79 ms.
#ifndef SPARC_LB_NT
#define SPARC_LB_NT 3
#endif
// A plane row of the look-back kernels: ``row_elems`` (wave-uniform element
// offset of the row's mode block) in scalar registers, the lane's V elements
// at ``lane_bytes`` in a vector register.
template <typename IO, int V>
__device__ __forceinline__ typename Raw<IO, V>::T lb_load(const void* base, int64_t row_elems,
                                                          uint32_t lane_bytes) {
  return ldn<typename Raw<IO, V>::T, (SPARC_LB_NT & 1) != 0>(
      base, wave_uniform(row_elems * static_cast<int64_t>(sizeof(IO))), lane_bytes);
}
template <typename IO, int V>
__device__ __forceinline__ void lb_store(void* base, int64_t row_elems, uint32_t lane_bytes,
                                         typename Raw<IO, V>::T v) {
  stn<typename Raw<IO, V>::T, (SPARC_LB_NT & 2) != 0>(
      base, wave_uniform(row_elems * static_cast<int64_t>(sizeof(IO))), lane_bytes, v);
}

// Look-back publication.  Aggregates and inclusive carries travel between
// workgroups (possibly on different XCDs) through sc1 stores and loads, the
// cache policy of agent-scope atomics (written through to, and read from, the
// device coherence point), here as wide vector accesses through a buffer
// resource at a wave-uniform base.  No access needs to be atomic: a consumer
// reads only after the producer's flag, which the producer stores after its
// data stores have completed.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t uniform_rsrc(const float* base, uint32_t bytes) {
  return make_rsrc(reinterpret_cast<const float*>(wave_uniform(reinterpret_cast<int64_t>(base))), bytes);
}
// A tile's aggregate, N floats per lane.  For N a multiple of 4 they are kept
// as 16-byte pieces at [piece][lane], so that each store and load instruction
// of the wave covers 1 KiB contiguously; else [lane][N].
template <int N>
__device__ __forceinline__ void agg_store(float* tile, int lane, const float (&v)[N]) {
  const __amdgpu_buffer_rsrc_t r = uniform_rsrc(tile, 64 * N * 4);
  if constexpr (N % 4 == 0) {
#pragma unroll
    for (int k = 0; k < N / 4; ++k) {
      const float t[4] = {v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]};
      buffer_store_f32<4, CPOL_SC1>(r, static_cast<uint32_t>((k * 64 + lane) * 16), t);
    }
  } else {
    buffer_store_f32<N, CPOL_SC1>(r, static_cast<uint32_t>(lane * N * 4), v);
  }
}
template <int N>
__device__ __forceinline__ void agg_load(const float* tile, int lane, float (&v)[N]) {
  const __amdgpu_buffer_rsrc_t r = uniform_rsrc(tile, 64 * N * 4);
  if constexpr (N % 4 == 0) {
#pragma unroll
    for (int k = 0; k < N / 4; ++k) {
      float t[4];
      buffer_load_f32<4, CPOL_SC1>(r, static_cast<uint32_t>((k * 64 + lane) * 16), t);
#pragma unroll
      for (int i = 0; i < 4; ++i) v[4 * k + i] = t[i];
    }
  } else {
    buffer_load_f32<N, CPOL_SC1>(r, static_cast<uint32_t>(lane * N * 4), v);
  }
}
// A lane's N <= 4 contiguous floats of a [..., M, NH] state plane (chunk
// states, backward carries); ``block`` is the mode block's first element.
template <int N>
__device__ __forceinline__ void state_store(float* block, int lane, const float (&v)[N]) {
  buffer_store_f32<N, CPOL_SC1>(uniform_rsrc(block, 64 * N * 4), static_cast<uint32_t>(lane * N * 4), v);
}
template <int N>
__device__ __forceinline__ void state_load(const float* block, int lane, float (&v)[N]) {
  buffer_load_f32<N, CPOL_SC1>(uniform_rsrc(block, 64 * N * 4), static_cast<uint32_t>(lane * N * 4), v);
}

template <typename T> struct IsBf16 : std::false_type {};
template <> struct IsBf16<bf16> : std::true_type {};

// ----- small complex helpers ----------------------------------------------
__device__ __forceinline__ void cmul(float ar, float ai, float br, float bi, float& cr, float& ci) {
  cr = ar * br - ai * bi;
  ci = ar * bi + ai * br;
}

// Per-lane agent-scope (sc1) loads and stores of a lane's N floats, 8 bytes at
// a time (the backward look-back: its register allocation under the 4-wave
// bound runs faster with these than with the wide accesses above).
template <int N>
__device__ __forceinline__ void load_agent_vec(const float* p, float (&o)[N]) {
  if constexpr (N % 2 == 0) {
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
      uint64_t u = load_agent(reinterpret_cast<const uint64_t*>(p) + i);
      o[2 * i] = __uint_as_float(static_cast<uint32_t>(u));
      o[2 * i + 1] = __uint_as_float(static_cast<uint32_t>(u >> 32));
    }
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) o[i] = __uint_as_float(load_agent(reinterpret_cast<const uint32_t*>(p) + i));
  }
}
template <int N>
__device__ __forceinline__ void store_agent_vec(float* p, const float (&v)[N]) {
  if constexpr (N % 2 == 0) {
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
      uint64_t u = static_cast<uint64_t>(__float_as_uint(v[2 * i])) |
                   (static_cast<uint64_t>(__float_as_uint(v[2 * i + 1])) << 32);
      store_agent(reinterpret_cast<uint64_t*>(p) + i, u);
    }
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) store_agent(reinterpret_cast<uint32_t*>(p) + i, __float_as_uint(v[i]));
  }
}

// The look-back walks its chain a window at a time.  Lane i reads the flag of
// chunk j + i * dir (positions outside the chain read as inclusive: the
// chain's end chunk always publishes an inclusive carry, so the walk never
// reaches them).  Returned, wave-uniform: the number n of consecutive chunks
// from j whose aggregates are published, and whether chunk j + n * dir holds
// an inclusive carry that ends the walk.  A whole window of aggregates is
// consumed per flag read, instead of one flag and one aggregate round trip
// per chunk, so few long chains still move their carry frontier at the rate
// their tiles finish.  Spins only while chunk j has published nothing, at most
// `limit` polls: then it sets *error and reports {0, inclusive, failed}, so
// that every wave still finishes; the caller then poisons its carry with NaN,
// so the failure shows in the outputs and gradients as well as in the error
// word.
constexpr int kLbLoads = 4;  // aggregates in flight per composition step (forward)
#ifndef SPARC_LB_BWD_LOADS
#define SPARC_LB_BWD_LOADS 1
#endif
constexpr int kLbLoadsBwd = SPARC_LB_BWD_LOADS;  // the same, backward (register-bound)
struct LbWindow {
  int n;
  bool incl;
  bool failed;  // the wait gave up: the carry it ends on is not valid
};
__device__ __forceinline__ LbWindow lb_window(const uint32_t* flags, int j, int dir, int n_chunks, uint32_t* error,
                                              uint32_t limit, int lane) {
  const int jl = j + lane * dir;
  const bool in_chain = jl >= 0 && jl < n_chunks;
  for (uint32_t it = 0; it < limit; ++it) {
    const uint32_t f = in_chain ? load_agent(flags + jl) : uint32_t(FLAG_INCLUSIVE);
    const uint64_t incl = __ballot(f == FLAG_INCLUSIVE);
    const uint64_t empty = __ballot(f == FLAG_EMPTY);
    const int fi = incl ? __builtin_ctzll(incl) : 64;
    const int fe = empty ? __builtin_ctzll(empty) : 64;
    if (fi == 0 || fe > 0) {
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      return fi < fe ? LbWindow{fi, true, false} : LbWindow{fe, false, false};
    }
    // once any wait of this launch has failed, stop waiting at all
    if ((it & 255u) == 255u && __builtin_amdgcn_readfirstlane(load_agent(error)) != 0u) break;
    __builtin_amdgcn_s_sleep(2);
  }
  store_agent(error, 1u);
  return LbWindow{0, true, true};
}

// ---------------------------------------------------------------------------
// Per-lane transition machinery
// ---------------------------------------------------------------------------
template <int TR, typename IO, int V, int GM>
struct TransitionLane {
  static constexpr bool CPLX = tr_kind(TR) != TR_REAL;
  static constexpr bool P1 = tr_kind(TR) == TR_P1;
  // number of distinct gate values per lane and step
  static constexpr int GV = (GM == GATE_MODE) ? V : 1;
  // number of distinct transition values per lane and step
  static constexpr int AV = (P1 || GM == GATE_MODE) ? V : 1;
  using GT = std::conditional_t<P1 || tr_g32(TR), float, IO>;  // gate dtype

  // P1 per-mode constants
  float nu[P1 ? V : 1], th[P1 ? V : 1], ct[P1 ? V : 1], st[P1 ? V : 1];

  __device__ __forceinline__ void init(const ScanArgs& p, int m0, bool ok) {
    if constexpr (P1) {
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const float nl = ok ? p.nu_log[m0 + v] : 0.0f;
        const float tl = ok ? p.theta_log[m0 + v] : 0.0f;
        nu[v] = expf(nl);
        th[v] = theta_rotation(tl, ct[v], st[v]);
      }
    }
  }

  // gate index of the lane's first mode
  __device__ __forceinline__ int64_t gate_index(const ScanArgs& p, int b, int t, int m0) const {
    const int64_t row = static_cast<int64_t>(b) * p.T + t;
    if constexpr (GM == GATE_MODE) return row * p.M + m0;
    else return row * p.G + m0 / p.gs;
  }

  __device__ __forceinline__ void load_gates(const ScanArgs& p, int64_t gi, float (&g0)[GV], float (&g1)[GV]) const {
    if constexpr (GM == GATE_MODE) {
      float tmp[V];
      unpack<GT, V>(load_raw<GT, V>(p.g0, gi), tmp);
#pragma unroll
      for (int v = 0; v < V; ++v) g0[v] = tmp[v];
      if constexpr (CPLX) {
        unpack<GT, V>(load_raw<GT, V>(p.g1, gi), tmp);
#pragma unroll
        for (int v = 0; v < V; ++v) g1[v] = tmp[v];
      } else {
#pragma unroll
        for (int v = 0; v < V; ++v) g1[v] = 0.0f;
      }
    } else {
      g0[0] = load1<GT>(p.g0, gi);
      g1[0] = CPLX ? load1<GT>(p.g1, gi) : 0.0f;
    }
  }

  // a = transition(g0, g1) for every distinct value
  __device__ __forceinline__ void transition(const float (&g0)[GV], const float (&g1)[GV],
                                             float (&ar)[AV], float (&ai)[AV]) const {
    if constexpr (P1) {
      const float E = fast_exp(g0[0]);  // GV == 1 for P1
      const float delta = g1[0];
#pragma unroll
      for (int v = 0; v < V; ++v) {
        // rho - 1 directly: for slow modes rho is within 1e-4 of 1, and
        // 1 - fp32(rho) would keep only a few bits of the phase increment
        const float em = expm1_nonpos(-nu[v] * E);
        const float rho = 1.0f + em;
        float sd, cd;
        sincos_quarter_or_half(-em * delta, sd, cd);
        ar[v] = rho * (ct[v] * cd - st[v] * sd);
        ai[v] = rho * (st[v] * cd + ct[v] * sd);
      }
    } else if constexpr (tr_kind(TR) == TR_POLAR) {
#pragma unroll
      for (int v = 0; v < AV; ++v) {
        float s, c;
        sincos_moderate(g1[v], s, c);
        ar[v] = g0[v] * c;
        ai[v] = g0[v] * s;
      }
    } else if constexpr (tr_kind(TR) == TR_CART) {
#pragma unroll
      for (int v = 0; v < AV; ++v) {
        ar[v] = g0[v];
        ai[v] = g1[v];
      }
    } else {
#pragma unroll
      for (int v = 0; v < AV; ++v) {
        ar[v] = g0[v];
        ai[v] = 0.0f;
      }
    }
  }

  // |delta*(1-rho)| <= pi/2 for the P1 controls (|delta| <= pi/2), but
  // eta/delta are caller data: reduce generally when out of the quarter range.
  __device__ __forceinline__ static void sincos_quarter_or_half(float x, float& s, float& c) {
    sincos_moderate(x, s, c);
  }
};

// ---------------------------------------------------------------------------
// Forward kernel
// ---------------------------------------------------------------------------
template <int TR, typename IO, int V, int GM, int S, int NW>
__global__ void __launch_bounds__(NW * 64)
scan_fwd_kernel(ScanArgs p) {
  using TL = TransitionLane<TR, IO, V, GM>;
  constexpr bool CPLX = TL::CPLX;
  constexpr int AV = TL::AV;
  constexpr int GV = TL::GV;
  constexpr int C = S * NW;
  constexpr int MB = 64 * V;
  constexpr int NQ = CPLX ? 4 : 2;   // (P re, P im, Q re, Q im) or (P, Q)
  constexpr int NH = CPLX ? 2 : 1;
  using RawT = typename Raw<IO, V>::T;

  __shared__ float s_pq[NW][NQ][V][64];
  __shared__ float s_start[NW][NH][V][64];
  __shared__ uint32_t s_tile;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));  // wave-uniform (scalar branches)
  if (threadIdx.x == 0) s_tile = atomicAdd(p.ticket, 1u);
  __syncthreads();
  const uint32_t tile = s_tile;
  const int chain = static_cast<int>(tile % static_cast<uint32_t>(p.n_chains));
  const int chunk = static_cast<int>(tile / static_cast<uint32_t>(p.n_chains));
  const int b = chain / p.n_mblocks;
  const int mb = chain - b * p.n_mblocks;
  const int m0 = mb * MB + lane * V;
  const bool lane_ok = m0 < p.M;
  const int mb0 = mb * MB;                                           // the block's first mode
  const uint32_t lane_bytes = static_cast<uint32_t>(lane * V * sizeof(IO));
  const int t0 = chunk * C + wave * S;
  const bool relu_out = CPLX && (p.flags & SPARC_FLAG_RELU_OUTPUT);
  const bool reset_first = (p.flags & SPARC_FLAG_RESET_FIRST) != 0;

  TL tl;
  tl.init(p, m0, lane_ok);

  // ---- load the sub-chunk: inputs, gates, transitions --------------------
  RawT wr_raw[S], wi_raw[S];
  float g0[S][GV], g1[S][GV];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const int t = t0 + s;
    const bool ok = lane_ok && t < p.T;
    const int64_t idx = (static_cast<int64_t>(b) * p.T + t) * p.M + mb0;  // row of the block
    if (ok) {
      wr_raw[s] = lb_load<IO, V>(p.w_re, idx, lane_bytes);
      if constexpr (CPLX) wi_raw[s] = lb_load<IO, V>(p.w_im, idx, lane_bytes);
      tl.load_gates(p, tl.gate_index(p, b, t, m0), g0[s], g1[s]);
    } else {
      float z[V] = {};
      wr_raw[s] = pack<IO, V>(z);
      if constexpr (CPLX) wi_raw[s] = wr_raw[s];
#pragma unroll
      for (int v = 0; v < GV; ++v) { g0[s][v] = 0.0f; g1[s][v] = 0.0f; }
    }
  }
  float a_r[S][AV], a_i[S][AV];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const int t = t0 + s;
    tl.transition(g0[s], g1[s], a_r[s], a_i[s]);
    bool reset;
    if (p.segpos) reset = (t < p.T) && p.segpos[static_cast<int64_t>(b) * p.T + t] == 0;
    else reset = reset_first && t == 0;
    const bool ident = !(lane_ok && t < p.T);
#pragma unroll
    for (int v = 0; v < AV; ++v) {
      if (ident) { a_r[s][v] = 1.0f; a_i[s][v] = 0.0f; }
      if (reset) { a_r[s][v] = 0.0f; a_i[s][v] = 0.0f; }
    }
  }

  // ---- 1. local scan of the sub-chunk from a zero state ------------------
  float Pr[AV], Pi[AV], Qr[V], Qi[V];
#pragma unroll
  for (int v = 0; v < AV; ++v) { Pr[v] = 1.0f; Pi[v] = 0.0f; }
#pragma unroll
  for (int v = 0; v < V; ++v) { Qr[v] = 0.0f; Qi[v] = 0.0f; }
#pragma unroll
  for (int s = 0; s < S; ++s) {
    float wr[V], wi[V];
    unpack<IO, V>(wr_raw[s], wr);
    if constexpr (CPLX) unpack<IO, V>(wi_raw[s], wi);
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int av = AV == 1 ? 0 : v;
      if constexpr (CPLX) {
        const float nr = a_r[s][av] * Qr[v] - a_i[s][av] * Qi[v] + wr[v];
        const float ni = a_i[s][av] * Qr[v] + a_r[s][av] * Qi[v] + wi[v];
        Qr[v] = nr;
        Qi[v] = ni;
      } else {
        Qr[v] = a_r[s][av] * Qr[v] + wr[v];
      }
    }
#pragma unroll
    for (int v = 0; v < AV; ++v) {
      if constexpr (CPLX) {
        float nr, ni;
        cmul(a_r[s][v], a_i[s][v], Pr[v], Pi[v], nr, ni);
        Pr[v] = nr;
        Pi[v] = ni;
      } else {
        Pr[v] = a_r[s][v] * Pr[v];
      }
    }
  }
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int av = AV == 1 ? 0 : v;
    s_pq[wave][0][v][lane] = Pr[av];
    if constexpr (CPLX) {
      s_pq[wave][1][v][lane] = Pi[av];
      s_pq[wave][2][v][lane] = Qr[v];
      s_pq[wave][3][v][lane] = Qi[v];
    } else {
      s_pq[wave][1][v][lane] = Qr[v];
    }
  }
  __syncthreads();

  // ---- 2./3. tile aggregate, look-back, inclusive carry (wave 0) ---------
  if (wave == 0) {
    float TPr[V], TPi[V], TQr[V], TQi[V];
#pragma unroll
    for (int v = 0; v < V; ++v) { TPr[v] = 1.0f; TPi[v] = 0.0f; TQr[v] = 0.0f; TQi[v] = 0.0f; }
#pragma unroll
    for (int k = 0; k < NW; ++k) {
#pragma unroll
      for (int v = 0; v < V; ++v) {
        if constexpr (CPLX) {
          const float pr = s_pq[k][0][v][lane], pi = s_pq[k][1][v][lane];
          const float qr = s_pq[k][2][v][lane], qi = s_pq[k][3][v][lane];
          float nr, ni;
          cmul(pr, pi, TQr[v], TQi[v], nr, ni);
          TQr[v] = nr + qr;
          TQi[v] = ni + qi;
          cmul(pr, pi, TPr[v], TPi[v], nr, ni);
          TPr[v] = nr;
          TPi[v] = ni;
        } else {
          const float pr = s_pq[k][0][v][lane], qr = s_pq[k][1][v][lane];
          TQr[v] = pr * TQr[v] + qr;
          TPr[v] = pr * TPr[v];
        }
      }
    }
    float cr[V], ci[V];
    if (chunk == 0) {
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const int64_t hi = static_cast<int64_t>(b) * p.M + m0 + v;
        cr[v] = (p.h0_re && lane_ok) ? p.h0_re[hi] : 0.0f;
        ci[v] = (CPLX && p.h0_im && lane_ok) ? p.h0_im[hi] : 0.0f;
      }
    } else {
      // publish the aggregate of this tile
      float* my_agg = p.agg + (static_cast<int64_t>(chain) * p.n_chunks + chunk) * MB * NQ;
      float pv[V * NQ];
#pragma unroll
      for (int v = 0; v < V; ++v) {
        pv[v * NQ + 0] = TPr[v];
        if constexpr (CPLX) {
          pv[v * NQ + 1] = TPi[v];
          pv[v * NQ + 2] = TQr[v];
          pv[v * NQ + 3] = TQi[v];
        } else {
          pv[v * NQ + 1] = TQr[v];
        }
      }
      agg_store<V * NQ>(my_agg, lane, pv);
      wait_stores_complete();
      if (lane == 0) store_agent(p.flagv + static_cast<int64_t>(chain) * p.n_chunks + chunk, uint32_t(FLAG_AGGREGATE));
      // look back: X = composition of the aggregates of chunks j+1 .. chunk-1
      float Xpr[V], Xpi[V], Xqr[V], Xqi[V];
#pragma unroll
      for (int v = 0; v < V; ++v) { Xpr[v] = 1.0f; Xpi[v] = 0.0f; Xqr[v] = 0.0f; Xqi[v] = 0.0f; }
      int j = chunk - 1;
      const uint32_t* chain_flags = p.flagv + static_cast<int64_t>(chain) * p.n_chunks;
      while (true) {
        const LbWindow w = lb_window(chain_flags, j, -1, p.n_chunks, p.error, p.spin_limit, lane);
        // compose the aggregates of chunks j, j-1, ..., j-w.n+1 (nearest
        // first), kLbLoads loads in flight at a time
        for (int base = 0; base < w.n; base += kLbLoads) {
          float q[kLbLoads][V * NQ];
#pragma unroll
          for (int u = 0; u < kLbLoads; ++u)
            if (base + u < w.n)
              agg_load<V * NQ>(p.agg + (static_cast<int64_t>(chain) * p.n_chunks + (j - base - u)) * MB * NQ, lane,
                               q[u]);
#pragma unroll
          for (int u = 0; u < kLbLoads; ++u) {
            if (base + u >= w.n) break;
#pragma unroll
            for (int v = 0; v < V; ++v) {
              if constexpr (CPLX) {
                float nr, ni;
                cmul(Xpr[v], Xpi[v], q[u][v * 4 + 2], q[u][v * 4 + 3], nr, ni);
                Xqr[v] += nr;
                Xqi[v] += ni;
                cmul(Xpr[v], Xpi[v], q[u][v * 4 + 0], q[u][v * 4 + 1], nr, ni);
                Xpr[v] = nr;
                Xpi[v] = ni;
              } else {
                Xqr[v] += Xpr[v] * q[u][v * 2 + 1];
                Xpr[v] *= q[u][v * 2 + 0];
              }
            }
          }
        }
        j -= w.n;
        if (w.incl) {
          float h[V * NH] = {};
          if (lane_ok && j >= 0)
            state_load<V * NH>(p.chunk_state + ((static_cast<int64_t>(b) * p.n_chunks + j) * p.M + mb0) * NH, lane, h);
#pragma unroll
          for (int v = 0; v < V; ++v) {
            if constexpr (CPLX) {
              float nr, ni;
              cmul(Xpr[v], Xpi[v], h[2 * v], h[2 * v + 1], nr, ni);
              cr[v] = nr + Xqr[v];
              ci[v] = ni + Xqi[v];
            } else {
              cr[v] = Xpr[v] * h[v] + Xqr[v];
              ci[v] = 0.0f;
            }
          }
          if (w.failed) {  // gave up waiting: make the failure visible downstream
#pragma unroll
            for (int v = 0; v < V; ++v) {
              cr[v] = __builtin_nanf("");
              if constexpr (CPLX) ci[v] = __builtin_nanf("");
            }
          }
          break;
        }
      }
    }
    // start state of every wave, and the inclusive carry of the tile
#pragma unroll
    for (int k = 0; k < NW; ++k) {
#pragma unroll
      for (int v = 0; v < V; ++v) {
        s_start[k][0][v][lane] = cr[v];
        if constexpr (CPLX) s_start[k][1][v][lane] = ci[v];
        if constexpr (CPLX) {
          const float pr = s_pq[k][0][v][lane], pi = s_pq[k][1][v][lane];
          const float qr = s_pq[k][2][v][lane], qi = s_pq[k][3][v][lane];
          float nr, ni;
          cmul(pr, pi, cr[v], ci[v], nr, ni);
          cr[v] = nr + qr;
          ci[v] = ni + qi;
        } else {
          cr[v] = s_pq[k][0][v][lane] * cr[v] + s_pq[k][1][v][lane];
        }
      }
    }
    if (lane_ok) {
      float h[V * NH];
#pragma unroll
      for (int v = 0; v < V; ++v) {
        if constexpr (CPLX) { h[2 * v] = cr[v]; h[2 * v + 1] = ci[v]; }
        else h[v] = cr[v];
      }
      state_store<V * NH>(p.chunk_state + ((static_cast<int64_t>(b) * p.n_chunks + chunk) * p.M + mb0) * NH, lane, h);
    }
    wait_stores_complete();
    if (lane == 0) store_agent(p.flagv + static_cast<int64_t>(chain) * p.n_chunks + chunk, uint32_t(FLAG_INCLUSIVE));
  }
  __syncthreads();

  // ---- 4. replay the sub-chunk from its start state and store -------------
  float hr[V], hi[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    hr[v] = s_start[wave][0][v][lane];
    hi[v] = CPLX ? s_start[wave][1][v][lane] : 0.0f;
  }
  if (!lane_ok) return;
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const int t = t0 + s;
    float wr[V], wi[V];
    unpack<IO, V>(wr_raw[s], wr);
    if constexpr (CPLX) unpack<IO, V>(wi_raw[s], wi);
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int av = AV == 1 ? 0 : v;
      if constexpr (CPLX) {
        const float nr = a_r[s][av] * hr[v] - a_i[s][av] * hi[v] + wr[v];
        const float ni = a_i[s][av] * hr[v] + a_r[s][av] * hi[v] + wi[v];
        hr[v] = nr;
        hi[v] = ni;
      } else {
        hr[v] = a_r[s][av] * hr[v] + wr[v];
      }
    }
    if (t < p.T) {
      const int64_t row = static_cast<int64_t>(b) * p.T + t;
      if (relu_out) {
        float rr[V], ri[V];
#pragma unroll
        for (int v = 0; v < V; ++v) { rr[v] = fmaxf(hr[v], 0.0f); ri[v] = fmaxf(hi[v], 0.0f); }
        lb_store<IO, V>(p.y_re, row * 2 * p.M + mb0, lane_bytes, pack<IO, V>(rr));
        lb_store<IO, V>(p.y_re, row * 2 * p.M + p.M + mb0, lane_bytes, pack<IO, V>(ri));
      } else {
        lb_store<IO, V>(p.y_re, row * p.M + mb0, lane_bytes, pack<IO, V>(hr));
        if constexpr (CPLX) lb_store<IO, V>(p.y_im, row * p.M + mb0, lane_bytes, pack<IO, V>(hi));
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Backward kernel
// ---------------------------------------------------------------------------
// SAVED: the states h_{t-1} come from the forward's saved output y (no relu
// epilogue) instead of being recomputed from w and the chunk states, so the
// tile skips the forward maps, their composition and the state replay.
// SAVED backward: load the states after the look-back (1) or with dy (0)
#ifndef SPARC_LB_SAVED_LATE
#define SPARC_LB_SAVED_LATE 1
#endif
// Waves per SIMD the SAVED backward is compiled for: 4, two workgroups per
// CU.  Real scans fit it without spills (90 registers; B=4, T=65536, M=4096
// fp32: 2.37 ms, against 2.87 ms at one workgroup per CU).  Polar and
// cartesian scans spill 6-12 registers under it and still gain (polar bf16,
// B=1, T=65536, M=2048: 1.00 -> 0.70 ms); P1 with two modes per lane would
// spill 68-118 and keeps the compiler's choice.
#ifndef SPARC_LB_BWD_WAVES
#define SPARC_LB_BWD_WAVES 4
#endif
#ifndef SPARC_LB_BWD_WAVES_CPLX
#define SPARC_LB_BWD_WAVES_CPLX 4
#endif
template <int TR, typename IO, int V, int GM, int S, int NW, bool SAVED>
__global__ void __launch_bounds__(NW * 64, !SAVED                      ? 1
                                           : tr_kind(TR) == TR_REAL ? SPARC_LB_BWD_WAVES
                                           : tr_kind(TR) == TR_P1   ? 1
                                                                    : SPARC_LB_BWD_WAVES_CPLX)
scan_bwd_kernel(ScanArgs p) {
  using TL = TransitionLane<TR, IO, V, GM>;
  using GT = typename TL::GT;
  constexpr bool CPLX = TL::CPLX;
  constexpr bool P1 = tr_kind(TR) == TR_P1;
  constexpr int AV = TL::AV;
  constexpr int GV = TL::GV;
  constexpr int C = S * NW;
  constexpr int MB = 64 * V;
  constexpr int NQ = CPLX ? 4 : 2;
  constexpr int NH = CPLX ? 2 : 1;
  using RawT = typename Raw<IO, V>::T;

  __shared__ float s_pq[NW][NQ][V][64];
  __shared__ float s_start[NW][NH][V][64];
  __shared__ float s_par[P1 ? NW : 1][2][V][64];   // P1 parameter-gradient partials
  __shared__ uint32_t s_tile;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));  // wave-uniform (scalar branches)
  if (threadIdx.x == 0) s_tile = atomicAdd(p.ticket, 1u);
  __syncthreads();
  const uint32_t tile = s_tile;
  const int chain = static_cast<int>(tile % static_cast<uint32_t>(p.n_chains));
  const int chunk = p.n_chunks - 1 - static_cast<int>(tile / static_cast<uint32_t>(p.n_chains));
  const int b = chain / p.n_mblocks;
  const int mb = chain - b * p.n_mblocks;
  const int m0 = mb * MB + lane * V;
  const bool lane_ok = m0 < p.M;
  const int mb0 = mb * MB;                                           // the block's first mode
  const uint32_t lane_bytes = static_cast<uint32_t>(lane * V * sizeof(IO));
  const int t0 = chunk * C + wave * S;
  const bool relu_out = CPLX && (p.flags & SPARC_FLAG_RELU_OUTPUT);
  const bool reset_first = (p.flags & SPARC_FLAG_RESET_FIRST) != 0;

  TL tl;
  tl.init(p, m0, lane_ok);

  // ---- loads ----------------------------------------------------------------
  RawT wr_raw[S], wi_raw[S], dr_raw[S], di_raw[S];
  float g0[S][GV], g1[S][GV];
  bool rst[S];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const int t = t0 + s;
    const bool ok = lane_ok && t < p.T;
    const int64_t row = static_cast<int64_t>(b) * p.T + t;
    const int64_t idx = row * p.M + mb0;  // row of the block
    if (ok) {
      if constexpr (SAVED) {
        if constexpr (!SPARC_LB_SAVED_LATE) {  // y at t-1 (t = 0: own row, replaced by h0)
          const int64_t pidx = t > 0 ? idx - p.M : idx;
          wr_raw[s] = lb_load<IO, V>(p.y_re, pidx, lane_bytes);
          if constexpr (CPLX) wi_raw[s] = lb_load<IO, V>(p.y_im, pidx, lane_bytes);
        }
      } else {
        wr_raw[s] = lb_load<IO, V>(p.w_re, idx, lane_bytes);
        if constexpr (CPLX) wi_raw[s] = lb_load<IO, V>(p.w_im, idx, lane_bytes);
      }
      if (relu_out) {
        dr_raw[s] = lb_load<IO, V>(p.dy_re, row * 2 * p.M + mb0, lane_bytes);
        di_raw[s] = lb_load<IO, V>(p.dy_re, row * 2 * p.M + p.M + mb0, lane_bytes);
      } else {
        dr_raw[s] = lb_load<IO, V>(p.dy_re, idx, lane_bytes);
        if constexpr (CPLX) di_raw[s] = lb_load<IO, V>(p.dy_im, idx, lane_bytes);
      }
      tl.load_gates(p, tl.gate_index(p, b, t, m0), g0[s], g1[s]);
    } else {
      float z[V] = {};
      wr_raw[s] = pack<IO, V>(z);
      wi_raw[s] = wr_raw[s];
      dr_raw[s] = wr_raw[s];
      di_raw[s] = wr_raw[s];
#pragma unroll
      for (int v = 0; v < GV; ++v) { g0[s][v] = 0.0f; g1[s][v] = 0.0f; }
    }
    if (p.segpos) rst[s] = (t < p.T) && p.segpos[row] == 0;
    else rst[s] = reset_first && t == 0;
  }
  float a_r[S][AV], a_i[S][AV];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const int t = t0 + s;
    tl.transition(g0[s], g1[s], a_r[s], a_i[s]);
    const bool ident = !(lane_ok && t < p.T);
#pragma unroll
    for (int v = 0; v < AV; ++v) {
      if (ident) { a_r[s][v] = 1.0f; a_i[s][v] = 0.0f; }
      if (rst[s]) { a_r[s][v] = 0.0f; a_i[s][v] = 0.0f; }
    }
  }

  // ---- forward sub-chunk maps (identical arithmetic to the forward kernel) --
  if constexpr (!SAVED) {
    float Pr[AV], Pi[AV], Qr[V], Qi[V];
#pragma unroll
    for (int v = 0; v < AV; ++v) { Pr[v] = 1.0f; Pi[v] = 0.0f; }
#pragma unroll
    for (int v = 0; v < V; ++v) { Qr[v] = 0.0f; Qi[v] = 0.0f; }
#pragma unroll
    for (int s = 0; s < S; ++s) {
      float wr[V], wi[V];
      unpack<IO, V>(wr_raw[s], wr);
      if constexpr (CPLX) unpack<IO, V>(wi_raw[s], wi);
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const int av = AV == 1 ? 0 : v;
        if constexpr (CPLX) {
          const float nr = a_r[s][av] * Qr[v] - a_i[s][av] * Qi[v] + wr[v];
          const float ni = a_i[s][av] * Qr[v] + a_r[s][av] * Qi[v] + wi[v];
          Qr[v] = nr;
          Qi[v] = ni;
        } else {
          Qr[v] = a_r[s][av] * Qr[v] + wr[v];
        }
      }
#pragma unroll
      for (int v = 0; v < AV; ++v) {
        if constexpr (CPLX) {
          float nr, ni;
          cmul(a_r[s][v], a_i[s][v], Pr[v], Pi[v], nr, ni);
          Pr[v] = nr;
          Pi[v] = ni;
        } else {
          Pr[v] = a_r[s][v] * Pr[v];
        }
      }
    }
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int av = AV == 1 ? 0 : v;
      s_pq[wave][0][v][lane] = Pr[av];
      if constexpr (CPLX) {
        s_pq[wave][1][v][lane] = Pi[av];
        s_pq[wave][2][v][lane] = Qr[v];
        s_pq[wave][3][v][lane] = Qi[v];
      } else {
        s_pq[wave][1][v][lane] = Qr[v];
      }
    }
    __syncthreads();
  }
  if (!SAVED && wave == 0) {
    float cr[V], ci[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
      if (chunk == 0) {
        const int64_t hi = static_cast<int64_t>(b) * p.M + m0 + v;
        cr[v] = (p.h0_re && lane_ok) ? p.h0_re[hi] : 0.0f;
        ci[v] = (CPLX && p.h0_im && lane_ok) ? p.h0_im[hi] : 0.0f;
      } else {
        const int64_t ci_ = ((static_cast<int64_t>(b) * p.n_chunks + chunk - 1) * p.M + m0 + v) * NH;
        cr[v] = lane_ok ? p.chunk_state_in[ci_] : 0.0f;
        ci[v] = (CPLX && lane_ok) ? p.chunk_state_in[ci_ + 1] : 0.0f;
      }
    }
#pragma unroll
    for (int k = 0; k < NW; ++k) {
#pragma unroll
      for (int v = 0; v < V; ++v) {
        s_start[k][0][v][lane] = cr[v];
        if constexpr (CPLX) s_start[k][1][v][lane] = ci[v];
        if constexpr (CPLX) {
          const float pr = s_pq[k][0][v][lane], pi = s_pq[k][1][v][lane];
          const float qr = s_pq[k][2][v][lane], qi = s_pq[k][3][v][lane];
          float nr, ni;
          cmul(pr, pi, cr[v], ci[v], nr, ni);
          cr[v] = nr + qr;
          ci[v] = ni + qi;
        } else {
          cr[v] = s_pq[k][0][v][lane] * cr[v] + s_pq[k][1][v][lane];
        }
      }
    }
  }
  if constexpr (!SAVED) __syncthreads();

  // ---- recompute the states h_{t-1} of the sub-chunk; masked dy -------------
  float hpr[S][V], hpi[S][V];   // state before step s
  float dyr[S][V], dyi[S][V];   // effective output gradient at step s
  if constexpr (SAVED) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      float gr[V], gi[V];
      unpack<IO, V>(dr_raw[s], gr);
      if constexpr (CPLX) unpack<IO, V>(di_raw[s], gi);
#pragma unroll
      for (int v = 0; v < V; ++v) {
        dyr[s][v] = gr[v];
        dyi[s][v] = CPLX ? gi[v] : 0.0f;
      }
    }
  } else {
    float hr[V], hi[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
      hr[v] = s_start[wave][0][v][lane];
      hi[v] = CPLX ? s_start[wave][1][v][lane] : 0.0f;
    }
#pragma unroll
    for (int s = 0; s < S; ++s) {
      float wr[V], wi[V], gr[V], gi[V];
      unpack<IO, V>(wr_raw[s], wr);
      unpack<IO, V>(dr_raw[s], gr);
      if constexpr (CPLX) {
        unpack<IO, V>(wi_raw[s], wi);
        unpack<IO, V>(di_raw[s], gi);
      }
#pragma unroll
      for (int v = 0; v < V; ++v) {
        hpr[s][v] = hr[v];
        hpi[s][v] = CPLX ? hi[v] : 0.0f;
        const int av = AV == 1 ? 0 : v;
        if constexpr (CPLX) {
          const float nr = a_r[s][av] * hr[v] - a_i[s][av] * hi[v] + wr[v];
          const float ni = a_i[s][av] * hr[v] + a_r[s][av] * hi[v] + wi[v];
          hr[v] = nr;
          hi[v] = ni;
          dyr[s][v] = (relu_out && !(hr[v] > 0.0f)) ? 0.0f : gr[v];
          dyi[s][v] = (relu_out && !(hi[v] > 0.0f)) ? 0.0f : gi[v];
        } else {
          hr[v] = a_r[s][av] * hr[v] + wr[v];
          dyr[s][v] = gr[v];
          dyi[s][v] = 0.0f;
        }
      }
    }
  }

  // ---- reverse sub-chunk maps: xi_out = conj(P) xi_in + Q ------------------
  {
    float Xr[V], Xi[V];
    float Pr[AV], Pi[AV];  // SAVED: the sub-chunk's transition product, formed here
#pragma unroll
    for (int v = 0; v < V; ++v) { Xr[v] = 0.0f; Xi[v] = 0.0f; }
#pragma unroll
    for (int v = 0; v < AV; ++v) { Pr[v] = 1.0f; Pi[v] = 0.0f; }
#pragma unroll
    for (int s = S - 1; s >= 0; --s) {
      if constexpr (SAVED) {
#pragma unroll
        for (int v = 0; v < AV; ++v) {
          if constexpr (CPLX) {
            float nr, ni;
            cmul(a_r[s][v], a_i[s][v], Pr[v], Pi[v], nr, ni);
            Pr[v] = nr;
            Pi[v] = ni;
          } else {
            Pr[v] = a_r[s][v] * Pr[v];
          }
        }
      }
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const int av = AV == 1 ? 0 : v;
        const float lr = dyr[s][v] + Xr[v];
        const float li = dyi[s][v] + Xi[v];
        if constexpr (CPLX) {
          Xr[v] = a_r[s][av] * lr + a_i[s][av] * li;
          Xi[v] = -a_i[s][av] * lr + a_r[s][av] * li;
        } else {
          Xr[v] = a_r[s][av] * lr;
        }
      }
    }
    if constexpr (!SAVED) __syncthreads();  // s_pq of the forward maps is no longer read
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int av = AV == 1 ? 0 : v;
      if constexpr (CPLX) {
        // the product of conj(a) over the sub-chunk is conj of the forward product
        if constexpr (SAVED) {
          s_pq[wave][0][v][lane] = Pr[av];
          s_pq[wave][1][v][lane] = -Pi[av];
        } else {
          s_pq[wave][1][v][lane] = -s_pq[wave][1][v][lane];
        }
        s_pq[wave][2][v][lane] = Xr[v];
        s_pq[wave][3][v][lane] = Xi[v];
      } else {
        if constexpr (SAVED) s_pq[wave][0][v][lane] = Pr[av];
        s_pq[wave][1][v][lane] = Xr[v];
      }
    }
    (void)Pr;
    (void)Pi;
  }
  __syncthreads();

  // ---- tile reverse aggregate, look-back over later chunks (wave 0) -------
  if (wave == 0) {
    float TPr[V], TPi[V], TQr[V], TQi[V];
#pragma unroll
    for (int v = 0; v < V; ++v) { TPr[v] = 1.0f; TPi[v] = 0.0f; TQr[v] = 0.0f; TQi[v] = 0.0f; }
#pragma unroll
    for (int k = NW - 1; k >= 0; --k) {
#pragma unroll
      for (int v = 0; v < V; ++v) {
        if constexpr (CPLX) {
          const float pr = s_pq[k][0][v][lane], pi = s_pq[k][1][v][lane];
          const float qr = s_pq[k][2][v][lane], qi = s_pq[k][3][v][lane];
          float nr, ni;
          cmul(pr, pi, TQr[v], TQi[v], nr, ni);
          TQr[v] = nr + qr;
          TQi[v] = ni + qi;
          cmul(pr, pi, TPr[v], TPi[v], nr, ni);
          TPr[v] = nr;
          TPi[v] = ni;
        } else {
          const float pr = s_pq[k][0][v][lane], qr = s_pq[k][1][v][lane];
          TQr[v] = pr * TQr[v] + qr;
          TPr[v] = pr * TPr[v];
        }
      }
    }
    float cr[V], ci[V];
    if (chunk == p.n_chunks - 1) {
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const int64_t hi = static_cast<int64_t>(b) * p.M + m0 + v;
        cr[v] = (p.dlast_re && lane_ok) ? p.dlast_re[hi] : 0.0f;
        ci[v] = (CPLX && p.dlast_im && lane_ok) ? p.dlast_im[hi] : 0.0f;
      }
    } else {
      float* my_agg = p.agg + ((static_cast<int64_t>(chain) * p.n_chunks + chunk) * MB + lane * V) * NQ;
      float pv[V * NQ];
#pragma unroll
      for (int v = 0; v < V; ++v) {
        pv[v * NQ + 0] = TPr[v];
        if constexpr (CPLX) {
          pv[v * NQ + 1] = TPi[v];
          pv[v * NQ + 2] = TQr[v];
          pv[v * NQ + 3] = TQi[v];
        } else {
          pv[v * NQ + 1] = TQr[v];
        }
      }
      store_agent_vec<V * NQ>(my_agg, pv);
      wait_stores_complete();
      if (lane == 0) store_agent(p.flagv + static_cast<int64_t>(chain) * p.n_chunks + chunk, uint32_t(FLAG_AGGREGATE));
      float Xpr[V], Xpi[V], Xqr[V], Xqi[V];
#pragma unroll
      for (int v = 0; v < V; ++v) { Xpr[v] = 1.0f; Xpi[v] = 0.0f; Xqr[v] = 0.0f; Xqi[v] = 0.0f; }
      int j = chunk + 1;
      const uint32_t* chain_flags = p.flagv + static_cast<int64_t>(chain) * p.n_chunks;
      while (true) {
        const LbWindow w = lb_window(chain_flags, j, 1, p.n_chunks, p.error, p.spin_limit, lane);
        // compose the aggregates of chunks j, j+1, ..., j+w.n-1 (nearest
        // first), kLbLoadsBwd loads in flight at a time
        for (int base = 0; base < w.n; base += kLbLoadsBwd) {
          float q[kLbLoadsBwd][V * NQ];
#pragma unroll
          for (int u = 0; u < kLbLoadsBwd; ++u)
            if (base + u < w.n)
              load_agent_vec<V * NQ>(
                  p.agg + ((static_cast<int64_t>(chain) * p.n_chunks + (j + base + u)) * MB + lane * V) * NQ, q[u]);
#pragma unroll
          for (int u = 0; u < kLbLoadsBwd; ++u) {
            if (base + u >= w.n) break;
#pragma unroll
            for (int v = 0; v < V; ++v) {
              if constexpr (CPLX) {
                float nr, ni;
                cmul(Xpr[v], Xpi[v], q[u][v * 4 + 2], q[u][v * 4 + 3], nr, ni);
                Xqr[v] += nr;
                Xqi[v] += ni;
                cmul(Xpr[v], Xpi[v], q[u][v * 4 + 0], q[u][v * 4 + 1], nr, ni);
                Xpr[v] = nr;
                Xpi[v] = ni;
              } else {
                Xqr[v] += Xpr[v] * q[u][v * 2 + 1];
                Xpr[v] *= q[u][v * 2 + 0];
              }
            }
          }
        }
        j += w.n;
        if (w.incl) {
          float h[V * NH] = {};
          if (lane_ok && j < p.n_chunks)
            load_agent_vec<V * NH>(p.carry + ((static_cast<int64_t>(b) * p.n_chunks + j) * p.M + m0) * NH, h);
#pragma unroll
          for (int v = 0; v < V; ++v) {
            if constexpr (CPLX) {
              float nr, ni;
              cmul(Xpr[v], Xpi[v], h[2 * v], h[2 * v + 1], nr, ni);
              cr[v] = nr + Xqr[v];
              ci[v] = ni + Xqi[v];
            } else {
              cr[v] = Xpr[v] * h[v] + Xqr[v];
              ci[v] = 0.0f;
            }
          }
          if (w.failed) {  // gave up waiting: make the failure visible downstream
#pragma unroll
            for (int v = 0; v < V; ++v) {
              cr[v] = __builtin_nanf("");
              if constexpr (CPLX) ci[v] = __builtin_nanf("");
            }
          }
          break;
        }
      }
    }
    // incoming adjoint of every wave; the tile's outgoing adjoint
#pragma unroll
    for (int k = NW - 1; k >= 0; --k) {
#pragma unroll
      for (int v = 0; v < V; ++v) {
        s_start[k][0][v][lane] = cr[v];
        if constexpr (CPLX) s_start[k][1][v][lane] = ci[v];
        if constexpr (CPLX) {
          const float pr = s_pq[k][0][v][lane], pi = s_pq[k][1][v][lane];
          const float qr = s_pq[k][2][v][lane], qi = s_pq[k][3][v][lane];
          float nr, ni;
          cmul(pr, pi, cr[v], ci[v], nr, ni);
          cr[v] = nr + qr;
          ci[v] = ni + qi;
        } else {
          cr[v] = s_pq[k][0][v][lane] * cr[v] + s_pq[k][1][v][lane];
        }
      }
    }
    if (chunk > 0) {
      if (lane_ok) {
        float h[V * NH];
#pragma unroll
        for (int v = 0; v < V; ++v) {
          if constexpr (CPLX) { h[2 * v] = cr[v]; h[2 * v + 1] = ci[v]; }
          else h[v] = cr[v];
        }
        store_agent_vec<V * NH>(p.carry + ((static_cast<int64_t>(b) * p.n_chunks + chunk) * p.M + m0) * NH, h);
      }
      wait_stores_complete();
      if (lane == 0) store_agent(p.flagv + static_cast<int64_t>(chain) * p.n_chunks + chunk, uint32_t(FLAG_INCLUSIVE));
    } else if (lane_ok && p.dh0_re) {
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const int64_t hi = static_cast<int64_t>(b) * p.M + m0 + v;
        p.dh0_re[hi] = cr[v];
        if constexpr (CPLX) p.dh0_im[hi] = ci[v];
      }
    }
  }
  __syncthreads();

  // ---- final reverse pass: dw, transition gradients ------------------------
  if constexpr (SAVED) {  // the states before each step: y at t-1, h0 (or 0) at t = 0
#pragma unroll
    for (int s = 0; s < S && SPARC_LB_SAVED_LATE; ++s) {
      const int t = t0 + s;
      if (lane_ok && t < p.T) {
        // t = 0 re-reads its own row; the value is replaced by h0 below
        const int64_t pidx = (static_cast<int64_t>(b) * p.T + (t > 0 ? t - 1 : t)) * p.M + mb0;
        wr_raw[s] = lb_load<IO, V>(p.y_re, pidx, lane_bytes);
        if constexpr (CPLX) wi_raw[s] = lb_load<IO, V>(p.y_im, pidx, lane_bytes);
      } else {
        float z[V] = {};
        wr_raw[s] = pack<IO, V>(z);
        wi_raw[s] = wr_raw[s];
      }
    }
#pragma unroll
    for (int s = 0; s < S; ++s) {
      unpack<IO, V>(wr_raw[s], hpr[s]);
      if constexpr (CPLX) unpack<IO, V>(wi_raw[s], hpi[s]);
#pragma unroll
      for (int v = 0; v < V; ++v) {
        if constexpr (!CPLX) hpi[s][v] = 0.0f;
        if (t0 + s == 0) {
          const int64_t hi = static_cast<int64_t>(b) * p.M + m0 + v;
          hpr[s][v] = (p.h0_re && lane_ok) ? p.h0_re[hi] : 0.0f;
          if constexpr (CPLX) hpi[s][v] = (p.h0_im && lane_ok) ? p.h0_im[hi] : 0.0f;
        }
      }
    }
  }
  float Xr[V], Xi[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    Xr[v] = s_start[wave][0][v][lane];
    Xi[v] = CPLX ? s_start[wave][1][v][lane] : 0.0f;
  }
  float acc_nu[P1 ? V : 1], acc_th[P1 ? V : 1];
#pragma unroll
  for (int v = 0; v < (P1 ? V : 1); ++v) { acc_nu[v] = 0.0f; acc_th[v] = 0.0f; }

  // group reduction width (lanes) for GATE_LANE
  const int glanes = (GM == GATE_LANE) ? (p.gs / V) : 1;

#pragma unroll
  for (int s = S - 1; s >= 0; --s) {
    const int t = t0 + s;
    const bool t_ok = t < p.T;
    const int64_t row = static_cast<int64_t>(b) * p.T + t;
    float lr[V], li[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
      lr[v] = dyr[s][v] + Xr[v];
      li[v] = dyi[s][v] + Xi[v];
    }
    if (lane_ok && t_ok) {
      lb_store<IO, V>(p.dw_re, row * p.M + mb0, lane_bytes, pack<IO, V>(lr));
      if constexpr (CPLX) lb_store<IO, V>(p.dw_im, row * p.M + mb0, lane_bytes, pack<IO, V>(li));
    }
    // gradient of the transition: dL/da = lambda * conj(h_{t-1})
    float d0[GV], d1[GV];   // per-gate gradient contributions (summed over the lane's modes when GV == 1)
#pragma unroll
    for (int v = 0; v < GV; ++v) { d0[v] = 0.0f; d1[v] = 0.0f; }
    const bool live = lane_ok && t_ok && !rst[s];
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int av = AV == 1 ? 0 : v;
      const int gv = GV == 1 ? 0 : v;
      float gar, gai;
      if constexpr (CPLX) {
        gar = lr[v] * hpr[s][v] + li[v] * hpi[s][v];
        gai = -lr[v] * hpi[s][v] + li[v] * hpr[s][v];
      } else {
        gar = lr[v] * hpr[s][v];
        gai = 0.0f;
      }
      if (!live) { gar = 0.0f; gai = 0.0f; }
      if constexpr (P1) {
        const float E = fast_exp(g0[s][0]);
        const float delta = g1[s][0];
        const float lrad = -tl.nu[v] * E;
        const float em = expm1_nonpos(lrad);  // rho - 1 (as in the forward)
        const float rho = 1.0f + em;
        const float ar = a_r[s][av], ai = a_i[s][av];
        float radial = lrad * (gar * ar + gai * ai);
        const float phase = -gar * ai + gai * ar;
        acc_th[v] += tl.th[v] * phase;
        radial += (-lrad) * rho * delta * phase;
        acc_nu[v] += radial;
        d0[gv] += radial;
        d1[gv] -= phase * em;
      } else if constexpr (tr_kind(TR) == TR_POLAR) {
        const float r = g0[s][gv];
        const float ar = a_r[s][av], ai = a_i[s][av];
        // d|a|: (gar cos phi + gai sin phi); with a = r (cos, sin)
        float cphi, sphi;
        sincos_moderate(g1[s][gv], sphi, cphi);
        d0[gv] += gar * cphi + gai * sphi;
        d1[gv] += -gar * ai + gai * ar;
        (void)r;
      } else if constexpr (tr_kind(TR) == TR_CART) {
        d0[gv] += gar;
        d1[gv] += gai;
      } else {
        d0[gv] += gar;
      }
      // propagate: X = conj(a) * lambda
      if constexpr (CPLX) {
        Xr[v] = a_r[s][av] * lr[v] + a_i[s][av] * li[v];
        Xi[v] = -a_i[s][av] * lr[v] + a_r[s][av] * li[v];
      } else {
        Xr[v] = a_r[s][av] * lr[v];
      }
    }
    // store gate gradients
    if constexpr (GM == GATE_MODE) {
      if (lane_ok && t_ok) {
        store_raw<GT, V>(p.dg0, row * p.M + m0, pack<GT, V>(d0));
        if constexpr (CPLX) store_raw<GT, V>(p.dg1, row * p.M + m0, pack<GT, V>(d1));
      }
    } else if constexpr (GM == GATE_LANE) {
      // a runtime group width: one LDS permute per stage (at cfg3, one stage)
      // is cheaper here than group_sum's branch chain
      float x0 = d0[0], x1 = d1[0];
      for (int off = 1; off < glanes; off <<= 1) {
        x0 += __shfl_xor(x0, off, 64);
        if constexpr (CPLX) x1 += __shfl_xor(x1, off, 64);
      }
      if (lane_ok && t_ok && (lane & (glanes - 1)) == 0) {
        const int64_t gi = row * p.G + m0 / p.gs;
        store1<GT>(p.dg0, gi, x0);
        if constexpr (CPLX) store1<GT>(p.dg1, gi, x1);
      }
    } else {  // GATE_CROSS: wave partial over its modes -> [B*T, n_mblocks]
      const float x0 = group_sum(d0[0], 64);
      const float x1 = CPLX ? group_sum(d1[0], 64) : 0.0f;
      if (lane == 0 && t_ok) {
        p.part_g0[row * p.n_mblocks + mb] = x0;
        if constexpr (CPLX) p.part_g1[row * p.n_mblocks + mb] = x1;
      }
    }
  }

  // ---- P1 parameter gradients: sum the NW waves -> one partial per tile ----
  if constexpr (P1) {
#pragma unroll
    for (int v = 0; v < V; ++v) {
      s_par[wave][0][v][lane] = acc_nu[v];
      s_par[wave][1][v][lane] = acc_th[v];
    }
    __syncthreads();
    if (wave == 0 && lane_ok) {
      float pn[V], pt[V];
#pragma unroll
      for (int v = 0; v < V; ++v) { pn[v] = 0.0f; pt[v] = 0.0f; }
#pragma unroll
      for (int k = 0; k < NW; ++k) {
#pragma unroll
        for (int v = 0; v < V; ++v) {
          pn[v] += s_par[k][0][v][lane];
          pt[v] += s_par[k][1][v][lane];
        }
      }
      const int64_t prow = static_cast<int64_t>(b) * p.n_chunks + chunk;
#pragma unroll
      for (int v = 0; v < V; ++v) {
        p.part_nu[prow * p.M + m0 + v] = pn[v];
        p.part_theta[prow * p.M + m0 + v] = pt[v];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Chain-serial kernels: one workgroup owns one chain (b, mode block) and walks
// its chunks in order, so the carry between chunks never leaves the CU.  The
// loads of the next chunk are issued before the current chunk is scanned and
// stored (two register buffers).  No tickets, flags or look-back: used when
// there are enough chains to fill the GPU.
// ---------------------------------------------------------------------------
template <int TR, typename IO, int V, int GM, int S>
struct SubChunk {
  using TL = TransitionLane<TR, IO, V, GM>;
  using RawT = typename Raw<IO, V>::T;
  static constexpr bool CPLX = TL::CPLX;
  static constexpr int GV = TL::GV;
  RawT wr[S], wi[S];
  float g0[S][GV], g1[S][GV];

  // loads steps [t0, t0 + S) of row b for the lane's modes
  __device__ __forceinline__ void load(const ScanArgs& p, const TL& tl, int b, int t0, int m0, bool lane_ok) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int t = t0 + s;
      if (lane_ok && t < p.T) {
        const int64_t idx = (static_cast<int64_t>(b) * p.T + t) * p.M + m0;
        wr[s] = load_raw<IO, V>(p.w_re, idx);
        if constexpr (CPLX) wi[s] = load_raw<IO, V>(p.w_im, idx);
        tl.load_gates(p, tl.gate_index(p, b, t, m0), g0[s], g1[s]);
      } else {
        float z[V] = {};
        wr[s] = pack<IO, V>(z);
        wi[s] = wr[s];
#pragma unroll
        for (int v = 0; v < GV; ++v) { g0[s][v] = 0.0f; g1[s][v] = 0.0f; }
      }
    }
  }
};

// transitions of S steps starting at t0 (identity past T, zero at resets)
template <class TL, int S>
__device__ __forceinline__ void make_transitions(const ScanArgs& p, const TL& tl, int b, int t0, bool lane_ok,
                                                 bool reset_first, const float (&g0)[S][TL::GV],
                                                 const float (&g1)[S][TL::GV], float (&a_r)[S][TL::AV],
                                                 float (&a_i)[S][TL::AV], bool (&rst)[S]) {
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const int t = t0 + s;
    tl.transition(g0[s], g1[s], a_r[s], a_i[s]);
    if (p.segpos) rst[s] = (t < p.T) && p.segpos[static_cast<int64_t>(b) * p.T + t] == 0;
    else rst[s] = reset_first && t == 0;
    const bool ident = !(lane_ok && t < p.T);
#pragma unroll
    for (int v = 0; v < TL::AV; ++v) {
      if (ident) { a_r[s][v] = 1.0f; a_i[s][v] = 0.0f; }
      if (rst[s]) { a_r[s][v] = 0.0f; a_i[s][v] = 0.0f; }
    }
  }
}

// (P, Q) of S steps from a zero state, written to lds[NQ][V][64]
template <bool CPLX, typename IO, int V, int AV, int S, int NQ>
__device__ __forceinline__ void local_maps(const typename Raw<IO, V>::T (&wr)[S], const typename Raw<IO, V>::T (&wi)[S],
                                           const float (&a_r)[S][AV], const float (&a_i)[S][AV],
                                           float (&lds)[NQ][V][64], int lane) {
  float Pr[AV], Pi[AV], Qr[V], Qi[V];
#pragma unroll
  for (int v = 0; v < AV; ++v) { Pr[v] = 1.0f; Pi[v] = 0.0f; }
#pragma unroll
  for (int v = 0; v < V; ++v) { Qr[v] = 0.0f; Qi[v] = 0.0f; }
#pragma unroll
  for (int s = 0; s < S; ++s) {
    float xr[V], xi[V];
    unpack<IO, V>(wr[s], xr);
    if constexpr (CPLX) unpack<IO, V>(wi[s], xi);
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int av = AV == 1 ? 0 : v;
      if constexpr (CPLX) {
        const float nr = a_r[s][av] * Qr[v] - a_i[s][av] * Qi[v] + xr[v];
        const float ni = a_i[s][av] * Qr[v] + a_r[s][av] * Qi[v] + xi[v];
        Qr[v] = nr;
        Qi[v] = ni;
      } else {
        Qr[v] = a_r[s][av] * Qr[v] + xr[v];
      }
    }
#pragma unroll
    for (int v = 0; v < AV; ++v) {
      if constexpr (CPLX) {
        float nr, ni;
        cmul(a_r[s][v], a_i[s][v], Pr[v], Pi[v], nr, ni);
        Pr[v] = nr;
        Pi[v] = ni;
      } else {
        Pr[v] = a_r[s][v] * Pr[v];
      }
    }
  }
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int av = AV == 1 ? 0 : v;
    lds[0][v][lane] = Pr[av];
    if constexpr (CPLX) {
      lds[1][v][lane] = Pi[av];
      lds[2][v][lane] = Qr[v];
      lds[3][v][lane] = Qi[v];
    } else {
      lds[1][v][lane] = Qr[v];
    }
  }
}

// x <- P x + Q with (P, Q) from lds[NQ][V][64]
template <bool CPLX, int V, int NQ>
__device__ __forceinline__ void apply_map(const float (&lds)[NQ][V][64], int lane, float (&xr)[V], float (&xi)[V]) {
#pragma unroll
  for (int v = 0; v < V; ++v) {
    if constexpr (CPLX) {
      const float pr = lds[0][v][lane], pi = lds[1][v][lane];
      const float qr = lds[2][v][lane], qi = lds[3][v][lane];
      float nr, ni;
      cmul(pr, pi, xr[v], xi[v], nr, ni);
      xr[v] = nr + qr;
      xi[v] = ni + qi;
    } else {
      xr[v] = lds[0][v][lane] * xr[v] + lds[1][v][lane];
    }
  }
}

template <int TR, typename IO, int V, int GM, int S, int NW>
__global__ void __launch_bounds__(NW * 64)
chain_fwd_kernel(ScanArgs p) {
  if (blockIdx.x == 0 && threadIdx.x == 0) *p.error = 0u;  // no waits here: never an error
  using SC = SubChunk<TR, IO, V, GM, S>;
  using TL = typename SC::TL;
  constexpr bool CPLX = TL::CPLX;
  constexpr int AV = TL::AV;
  constexpr int C = S * NW;
  constexpr int MB = 64 * V;
  constexpr int NQ = CPLX ? 4 : 2;
  constexpr int NH = CPLX ? 2 : 1;
  __shared__ float s_pq[2][NW][NQ][V][64];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int chain = xcd_swizzle(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x));
  const int b = chain / p.n_mblocks;
  const int mb = chain - b * p.n_mblocks;
  const int m0 = mb * MB + lane * V;
  const bool lane_ok = m0 < p.M;
  const bool relu_out = CPLX && (p.flags & SPARC_FLAG_RELU_OUTPUT);
  const bool reset_first = (p.flags & SPARC_FLAG_RESET_FIRST) != 0;
  TL tl;
  tl.init(p, m0, lane_ok);

  float cr[V], ci[V];  // state entering the current chunk
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int64_t hi = static_cast<int64_t>(b) * p.M + m0 + v;
    cr[v] = (p.h0_re && lane_ok) ? p.h0_re[hi] : 0.0f;
    ci[v] = (CPLX && p.h0_im && lane_ok) ? p.h0_im[hi] : 0.0f;
  }
  SC buf[2];
  buf[0].load(p, tl, b, wave * S, m0, lane_ok);
  for (int c0 = 0; c0 < p.n_chunks; c0 += 2) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = c0 + h;
      if (c >= p.n_chunks) break;
      const int t0 = c * C + wave * S;
      if (c + 1 < p.n_chunks) buf[1 - h].load(p, tl, b, t0 + C, m0, lane_ok);
      float a_r[S][AV], a_i[S][AV];
      bool rst[S];
      make_transitions<TL, S>(p, tl, b, t0, lane_ok, reset_first, buf[h].g0, buf[h].g1, a_r, a_i, rst);
      local_maps<CPLX, IO, V, AV, S, NQ>(buf[h].wr, buf[h].wi, a_r, a_i, s_pq[h][wave], lane);
      __syncthreads();
      // start state of this wave, and the state after the chunk (same arithmetic in every wave)
      float sr[V], si[V];
#pragma unroll
      for (int k = 0; k < NW; ++k) {
        if (k == wave) {
#pragma unroll
          for (int v = 0; v < V; ++v) { sr[v] = cr[v]; si[v] = ci[v]; }
        }
        apply_map<CPLX, V, NQ>(s_pq[h][k], lane, cr, ci);
      }
      if (wave == 0 && lane_ok) {
        float hv[V * NH];
#pragma unroll
        for (int v = 0; v < V; ++v) {
          if constexpr (CPLX) { hv[2 * v] = cr[v]; hv[2 * v + 1] = ci[v]; }
          else hv[v] = cr[v];
        }
        float* dst = p.chunk_state + ((static_cast<int64_t>(b) * p.n_chunks + c) * p.M + m0) * NH;
#pragma unroll
        for (int i = 0; i < V * NH; ++i) dst[i] = hv[i];
      }
      // replay and store
      if (lane_ok) {
#pragma unroll
        for (int s = 0; s < S; ++s) {
          const int t = t0 + s;
          float xr[V], xi[V];
          unpack<IO, V>(buf[h].wr[s], xr);
          if constexpr (CPLX) unpack<IO, V>(buf[h].wi[s], xi);
#pragma unroll
          for (int v = 0; v < V; ++v) {
            const int av = AV == 1 ? 0 : v;
            if constexpr (CPLX) {
              const float nr = a_r[s][av] * sr[v] - a_i[s][av] * si[v] + xr[v];
              const float ni = a_i[s][av] * sr[v] + a_r[s][av] * si[v] + xi[v];
              sr[v] = nr;
              si[v] = ni;
            } else {
              sr[v] = a_r[s][av] * sr[v] + xr[v];
            }
          }
          if (t < p.T) {
            const int64_t row = static_cast<int64_t>(b) * p.T + t;
            if (relu_out) {
              float rr[V], ri[V];
#pragma unroll
              for (int v = 0; v < V; ++v) { rr[v] = fmaxf(sr[v], 0.0f); ri[v] = fmaxf(si[v], 0.0f); }
              store_raw<IO, V>(p.y_re, row * 2 * p.M + m0, pack<IO, V>(rr));
              store_raw<IO, V>(p.y_re, row * 2 * p.M + p.M + m0, pack<IO, V>(ri));
            } else {
              store_raw<IO, V>(p.y_re, row * p.M + m0, pack<IO, V>(sr));
              if constexpr (CPLX) store_raw<IO, V>(p.y_im, row * p.M + m0, pack<IO, V>(si));
            }
          }
        }
      }
    }
  }
}

template <int TR, typename IO, int V, int GM, int S, int NW>
__global__ void __launch_bounds__(NW * 64)
chain_bwd_kernel(ScanArgs p) {
  if (blockIdx.x == 0 && threadIdx.x == 0) *p.error = 0u;  // no waits here: never an error
  using SC = SubChunk<TR, IO, V, GM, S>;
  using TL = typename SC::TL;
  using GT = typename TL::GT;
  using RawT = typename Raw<IO, V>::T;
  constexpr bool CPLX = TL::CPLX;
  constexpr bool P1 = tr_kind(TR) == TR_P1;
  constexpr int AV = TL::AV;
  constexpr int GV = TL::GV;
  constexpr int C = S * NW;
  constexpr int MB = 64 * V;
  constexpr int NQ = CPLX ? 4 : 2;
  constexpr int NH = CPLX ? 2 : 1;
  __shared__ float s_fq[NW][NQ][V][64];   // forward sub-chunk maps
  __shared__ float s_rq[NW][NQ][V][64];   // reverse sub-chunk maps
  __shared__ float s_par[P1 ? NW : 1][2][V][64];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int chain = xcd_swizzle(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x));
  const int b = chain / p.n_mblocks;
  const int mb = chain - b * p.n_mblocks;
  const int m0 = mb * MB + lane * V;
  const bool lane_ok = m0 < p.M;
  const bool relu_out = CPLX && (p.flags & SPARC_FLAG_RELU_OUTPUT);
  const bool reset_first = (p.flags & SPARC_FLAG_RESET_FIRST) != 0;
  const int glanes = (GM == GATE_LANE) ? (p.gs / V) : 1;
  TL tl;
  tl.init(p, m0, lane_ok);

  float xr_c[V], xi_c[V];  // adjoint entering the current chunk from the future
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int64_t hi = static_cast<int64_t>(b) * p.M + m0 + v;
    xr_c[v] = (p.dlast_re && lane_ok) ? p.dlast_re[hi] : 0.0f;
    xi_c[v] = (CPLX && p.dlast_im && lane_ok) ? p.dlast_im[hi] : 0.0f;
  }
  float acc_nu[P1 ? V : 1], acc_th[P1 ? V : 1];
#pragma unroll
  for (int v = 0; v < (P1 ? V : 1); ++v) { acc_nu[v] = 0.0f; acc_th[v] = 0.0f; }

  SC buf[2];
  RawT dr[2][S], di[2][S];
  float hs[2][V * NH];  // state entering the chunk (saved by the forward)
  auto load_all = [&](int hb, int c) {
    const int t0 = c * C + wave * S;
    buf[hb].load(p, tl, b, t0, m0, lane_ok);
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int t = t0 + s;
      if (lane_ok && t < p.T) {
        const int64_t row = static_cast<int64_t>(b) * p.T + t;
        if (relu_out) {
          dr[hb][s] = load_raw<IO, V>(p.dy_re, row * 2 * p.M + m0);
          di[hb][s] = load_raw<IO, V>(p.dy_re, row * 2 * p.M + p.M + m0);
        } else {
          dr[hb][s] = load_raw<IO, V>(p.dy_re, row * p.M + m0);
          if constexpr (CPLX) di[hb][s] = load_raw<IO, V>(p.dy_im, row * p.M + m0);
        }
      } else {
        float z[V] = {};
        dr[hb][s] = pack<IO, V>(z);
        di[hb][s] = dr[hb][s];
      }
    }
#pragma unroll
    for (int v = 0; v < V; ++v) {
      if (c == 0) {
        const int64_t hi = static_cast<int64_t>(b) * p.M + m0 + v;
        hs[hb][v * NH] = (p.h0_re && lane_ok) ? p.h0_re[hi] : 0.0f;
        if constexpr (CPLX) hs[hb][v * NH + 1] = (p.h0_im && lane_ok) ? p.h0_im[hi] : 0.0f;
      } else {
        const int64_t ci_ = ((static_cast<int64_t>(b) * p.n_chunks + c - 1) * p.M + m0 + v) * NH;
        hs[hb][v * NH] = lane_ok ? p.chunk_state_in[ci_] : 0.0f;
        if constexpr (CPLX) hs[hb][v * NH + 1] = lane_ok ? p.chunk_state_in[ci_ + 1] : 0.0f;
      }
    }
  };

  load_all(0, p.n_chunks - 1);
  for (int c0 = p.n_chunks - 1; c0 >= 0; c0 -= 2) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = c0 - h;
      if (c < 0) break;
      const int t0 = c * C + wave * S;
      if (c - 1 >= 0) load_all(1 - h, c - 1);
      float a_r[S][AV], a_i[S][AV];
      bool rst[S];
      make_transitions<TL, S>(p, tl, b, t0, lane_ok, reset_first, buf[h].g0, buf[h].g1, a_r, a_i, rst);
      local_maps<CPLX, IO, V, AV, S, NQ>(buf[h].wr, buf[h].wi, a_r, a_i, s_fq[wave], lane);
      __syncthreads();  // B1: forward maps visible
      float hr[V], hi[V];
#pragma unroll
      for (int v = 0; v < V; ++v) { hr[v] = hs[h][v * NH]; hi[v] = CPLX ? hs[h][v * NH + 1] : 0.0f; }
      for (int k = 0; k < wave; ++k) apply_map<CPLX, V, NQ>(s_fq[k], lane, hr, hi);
      // recompute h_{t-1}; effective output gradient (relu mask from the recomputed state)
      float hpr[S][V], hpi[S][V], dyr[S][V], dyi[S][V];
#pragma unroll
      for (int s = 0; s < S; ++s) {
        float xw_r[V], xw_i[V], gr[V], gi[V];
        unpack<IO, V>(buf[h].wr[s], xw_r);
        unpack<IO, V>(dr[h][s], gr);
        if constexpr (CPLX) {
          unpack<IO, V>(buf[h].wi[s], xw_i);
          unpack<IO, V>(di[h][s], gi);
        }
#pragma unroll
        for (int v = 0; v < V; ++v) {
          hpr[s][v] = hr[v];
          hpi[s][v] = CPLX ? hi[v] : 0.0f;
          const int av = AV == 1 ? 0 : v;
          if constexpr (CPLX) {
            const float nr = a_r[s][av] * hr[v] - a_i[s][av] * hi[v] + xw_r[v];
            const float ni = a_i[s][av] * hr[v] + a_r[s][av] * hi[v] + xw_i[v];
            hr[v] = nr;
            hi[v] = ni;
            dyr[s][v] = (relu_out && !(hr[v] > 0.0f)) ? 0.0f : gr[v];
            dyi[s][v] = (relu_out && !(hi[v] > 0.0f)) ? 0.0f : gi[v];
          } else {
            hr[v] = a_r[s][av] * hr[v] + xw_r[v];
            dyr[s][v] = gr[v];
            dyi[s][v] = 0.0f;
          }
        }
      }
      // reverse map of the sub-chunk: xi_out = conj(prod a) xi_in + Q
      {
        float Xr[V], Xi[V];
#pragma unroll
        for (int v = 0; v < V; ++v) { Xr[v] = 0.0f; Xi[v] = 0.0f; }
#pragma unroll
        for (int s = S - 1; s >= 0; --s) {
#pragma unroll
          for (int v = 0; v < V; ++v) {
            const int av = AV == 1 ? 0 : v;
            const float lr = dyr[s][v] + Xr[v];
            const float li = dyi[s][v] + Xi[v];
            if constexpr (CPLX) {
              Xr[v] = a_r[s][av] * lr + a_i[s][av] * li;
              Xi[v] = -a_i[s][av] * lr + a_r[s][av] * li;
            } else {
              Xr[v] = a_r[s][av] * lr;
            }
          }
        }
#pragma unroll
        for (int v = 0; v < V; ++v) {
          s_rq[wave][0][v][lane] = s_fq[wave][0][v][lane];
          if constexpr (CPLX) {
            s_rq[wave][1][v][lane] = -s_fq[wave][1][v][lane];
            s_rq[wave][2][v][lane] = Xr[v];
            s_rq[wave][3][v][lane] = Xi[v];
          } else {
            s_rq[wave][1][v][lane] = Xr[v];
          }
        }
      }
      __syncthreads();  // B2: reverse maps visible
      // incoming adjoint of this wave; adjoint leaving the chunk (same in every wave)
      float Xr[V], Xi[V];
#pragma unroll
      for (int k = NW - 1; k >= 0; --k) {
        if (k == wave) {
#pragma unroll
          for (int v = 0; v < V; ++v) { Xr[v] = xr_c[v]; Xi[v] = xi_c[v]; }
        }
        apply_map<CPLX, V, NQ>(s_rq[k], lane, xr_c, xi_c);
      }
      // final reverse pass: dw, transition gradients
#pragma unroll
      for (int s = S - 1; s >= 0; --s) {
        const int t = t0 + s;
        const bool t_ok = t < p.T;
        const int64_t row = static_cast<int64_t>(b) * p.T + t;
        float lr[V], li[V];
#pragma unroll
        for (int v = 0; v < V; ++v) { lr[v] = dyr[s][v] + Xr[v]; li[v] = dyi[s][v] + Xi[v]; }
        if (lane_ok && t_ok) {
          store_raw<IO, V>(p.dw_re, row * p.M + m0, pack<IO, V>(lr));
          if constexpr (CPLX) store_raw<IO, V>(p.dw_im, row * p.M + m0, pack<IO, V>(li));
        }
        float d0[GV], d1[GV];
#pragma unroll
        for (int v = 0; v < GV; ++v) { d0[v] = 0.0f; d1[v] = 0.0f; }
        const bool live = lane_ok && t_ok && !rst[s];
#pragma unroll
        for (int v = 0; v < V; ++v) {
          const int av = AV == 1 ? 0 : v;
          const int gv = GV == 1 ? 0 : v;
          float gar, gai;
          if constexpr (CPLX) {
            gar = lr[v] * hpr[s][v] + li[v] * hpi[s][v];
            gai = -lr[v] * hpi[s][v] + li[v] * hpr[s][v];
          } else {
            gar = lr[v] * hpr[s][v];
            gai = 0.0f;
          }
          if (!live) { gar = 0.0f; gai = 0.0f; }
          if constexpr (P1) {
            const float E = fast_exp(buf[h].g0[s][0]);
            const float delta = buf[h].g1[s][0];
            const float lrad = -tl.nu[v] * E;
            const float em = expm1_nonpos(lrad);  // rho - 1 (as in the forward)
            const float rho = 1.0f + em;
            const float ar = a_r[s][av], ai = a_i[s][av];
            float radial = lrad * (gar * ar + gai * ai);
            const float phase = -gar * ai + gai * ar;
            acc_th[v] += tl.th[v] * phase;
            radial += (-lrad) * rho * delta * phase;
            acc_nu[v] += radial;
            d0[gv] += radial;
            d1[gv] -= phase * em;
          } else if constexpr (tr_kind(TR) == TR_POLAR) {
            const float ar = a_r[s][av], ai = a_i[s][av];
            float cphi, sphi;
            sincos_moderate(buf[h].g1[s][gv], sphi, cphi);
            d0[gv] += gar * cphi + gai * sphi;
            d1[gv] += -gar * ai + gai * ar;
          } else if constexpr (tr_kind(TR) == TR_CART) {
            d0[gv] += gar;
            d1[gv] += gai;
          } else {
            d0[gv] += gar;
          }
          if constexpr (CPLX) {
            const float nr = a_r[s][av] * lr[v] + a_i[s][av] * li[v];
            const float ni = -a_i[s][av] * lr[v] + a_r[s][av] * li[v];
            Xr[v] = nr;
            Xi[v] = ni;
          } else {
            Xr[v] = a_r[s][av] * lr[v];
          }
        }
        if constexpr (GM == GATE_MODE) {
          if (lane_ok && t_ok) {
            store_raw<GT, V>(p.dg0, row * p.M + m0, pack<GT, V>(d0));
            if constexpr (CPLX) store_raw<GT, V>(p.dg1, row * p.M + m0, pack<GT, V>(d1));
          }
        } else if constexpr (GM == GATE_LANE) {
          float x0 = d0[0], x1 = d1[0];
          for (int off = 1; off < glanes; off <<= 1) {
            x0 += __shfl_xor(x0, off, 64);
            if constexpr (CPLX) x1 += __shfl_xor(x1, off, 64);
          }
          if (lane_ok && t_ok && (lane & (glanes - 1)) == 0) {
            const int64_t gi = row * p.G + m0 / p.gs;
            store1<GT>(p.dg0, gi, x0);
            if constexpr (CPLX) store1<GT>(p.dg1, gi, x1);
          }
        } else {
          const float x0 = group_sum(d0[0], 64);
          const float x1 = CPLX ? group_sum(d1[0], 64) : 0.0f;
          if (lane == 0 && t_ok) {
            p.part_g0[row * p.n_mblocks + mb] = x0;
            if constexpr (CPLX) p.part_g1[row * p.n_mblocks + mb] = x1;
          }
        }
      }
    }
  }
  if (wave == 0 && lane_ok && p.dh0_re) {
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int64_t hi = static_cast<int64_t>(b) * p.M + m0 + v;
      p.dh0_re[hi] = xr_c[v];
      if constexpr (CPLX) p.dh0_im[hi] = xi_c[v];
    }
  }
  if constexpr (P1) {
#pragma unroll
    for (int v = 0; v < V; ++v) {
      s_par[wave][0][v][lane] = acc_nu[v];
      s_par[wave][1][v][lane] = acc_th[v];
    }
    __syncthreads();
    if (wave == 0 && lane_ok) {
      float pn[V], pt[V];
#pragma unroll
      for (int v = 0; v < V; ++v) { pn[v] = 0.0f; pt[v] = 0.0f; }
      for (int k = 0; k < NW; ++k) {
#pragma unroll
        for (int v = 0; v < V; ++v) { pn[v] += s_par[k][0][v][lane]; pt[v] += s_par[k][1][v][lane]; }
      }
#pragma unroll
      for (int v = 0; v < V; ++v) {
        p.part_nu[static_cast<int64_t>(b) * p.M + m0 + v] = pn[v];
        p.part_theta[static_cast<int64_t>(b) * p.M + m0 + v] = pt[v];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Fast chain-serial kernels for gates shared by the lanes of a group
// (GATE_LANE; polar, cartesian and real transitions; at most 16 gate groups
// per wave).  Same decomposition as the chain kernels above, plus:
//   * each transition a(step, group) is computed once, by one lane, and
//     shared through a per-wave LDS table (instead of by every lane of the
//     group); steps past T and reset steps are folded into that table, so
//     the inner loops carry no per-step selects;
//   * addresses are a wave-uniform running byte offset (scalar registers)
//     plus a fixed per-lane byte offset;
//   * the relu(cat) epilogue is a template parameter;
//   * gate gradients are summed over the lanes of a group with DPP lane
//     permutations (no LDS round trip);
//   * the carry entering each chunk lives in LDS; wave k composes only the
//     maps of waves 0..k-1, the last wave produces the next carry.
// ---------------------------------------------------------------------------
constexpr int kFastMaxGpw = 16;  // gate groups per wave handled by the fast kernels


constexpr int fast_rounds(int S) { return (S * kFastMaxGpw + 63) / 64; }

// Raw gate bits (and segment positions) of the (step, group) pairs of one
// block of S steps; lane l owns pairs l, l + 64, ...  (pair = step * gpw +
// group).  They are loaded a block ahead and stay raw until fill_tab converts
// them: a conversion right after the load would make the wave wait for it,
// and with it for every plane load of the prefetch issued just before.
template <int S>
struct GateBlock {
  uint32_t g0[fast_rounds(S)], g1[fast_rounds(S)];
  int32_t pos[fast_rounds(S)];
};

template <typename IO>
__device__ __forceinline__ uint32_t load_bits(const void* base, int64_t index) {
  if constexpr (sizeof(IO) == 4) return static_cast<const uint32_t*>(base)[index];
  else return static_cast<const uint16_t*>(base)[index];
}
template <typename IO>
__device__ __forceinline__ float bits_to_float(uint32_t bits) {
  if constexpr (sizeof(IO) == 4) return __uint_as_float(bits);
  else return __uint_as_float(bits << 16);
}

// Every lane loads: pairs outside the tensors (steps past T, groups past G in
// the last mode block, rounds past S * gpw) read element 0, and fill_tab
// discards them.
template <int TR, typename IO, int S>
__device__ __forceinline__ void load_gate_pairs(const ScanArgs& p, int b, int t0, int g_base, int gpw, int lane,
                                                GateBlock<S>& gb) {
#pragma unroll
  for (int r = 0; r < fast_rounds(S); ++r) {
    const int idx = r * 64 + lane;
    const int step = idx / gpw;
    const int t = t0 + step;
    const int g = g_base + idx - step * gpw;
    const bool in_t = idx < S * gpw && t < p.T;
    const int64_t row = static_cast<int64_t>(b) * p.T + t;
    const int64_t gi = (in_t && g < p.G) ? row * p.G + g : 0;
    gb.g0[r] = load_bits<IO>(p.g0, gi);
    if constexpr (TR != TR_REAL) gb.g1[r] = load_bits<IO>(p.g1, gi);
    if (p.segpos) gb.pos[r] = p.segpos[in_t ? row : 0];
  }
}

// tab[pair] = (ar, ai[, cos phi, sin phi]); identity past T, zero at resets
// and for groups past G.  Returns the lane's reset pairs as a bit mask (bit r:
// pair r * 64 + lane).
template <int TR, typename IO, int S, int TW>
__device__ __forceinline__ uint32_t fill_tab(const ScanArgs& p, int t0, int g_base, int gpw, int lane,
                                             bool reset_first, const GateBlock<S>& gb, float* tab) {
  uint32_t rmask = 0u;
#pragma unroll
  for (int r = 0; r < fast_rounds(S); ++r) {
    const int idx = r * 64 + lane;
    if (idx < S * gpw) {
      const int step = idx / gpw;
      const int t = t0 + step;
      const bool g_ok = g_base + idx - step * gpw < p.G;
      float ar = 1.0f, ai = 0.0f, cp = 1.0f, sp = 0.0f;
      if (t < p.T) {
        const float v0 = g_ok ? bits_to_float<IO>(gb.g0[r]) : 0.0f;
        const float v1 = (TR != TR_REAL && g_ok) ? bits_to_float<IO>(gb.g1[r]) : 0.0f;
        if constexpr (TR == TR_POLAR) {
          sincos_moderate(v1, sp, cp);
          ar = v0 * cp;
          ai = v0 * sp;
        } else if constexpr (TR == TR_CART) {
          ar = v0;
          ai = v1;
        } else {
          ar = v0;
        }
        const bool reset = p.segpos ? (gb.pos[r] == 0) : (reset_first && t == 0);
        if (reset) {
          ar = 0.0f;
          ai = 0.0f;
          rmask |= 1u << r;
        }
      }
      float* e = tab + idx * TW;
      e[0] = ar;
      if constexpr (TW > 1) e[1] = ai;
      if constexpr (TW > 2) { e[2] = cp; e[3] = sp; }
    }
  }
  return rmask;
}

template <int TR, typename IO, int V, int S, int NW, bool RELU>
__global__ void __launch_bounds__(NW * 64, 4)
chain_fwd_fast_kernel(ScanArgs p) {
  static_assert(!tr_g32(TR), "lane-shared kernels read gates in the I/O dtype");
  if (blockIdx.x == 0 && threadIdx.x == 0) *p.error = 0u;  // no waits here: never an error
  constexpr bool CPLX = TR != TR_REAL;
  constexpr int C = S * NW;
  constexpr int MB = 64 * V;
  constexpr int NH = CPLX ? 2 : 1;
  constexpr int TW = CPLX ? 2 : 1;
  constexpr int ESZ = sizeof(IO);
  using RawT = typename Raw<IO, V>::T;
  __shared__ float s_p[2][NW][NH][64];
  __shared__ float s_q[2][NW][NH][V][64];
  __shared__ float s_carry[2][NH][V][64];
  __shared__ float s_tab[NW][S * kFastMaxGpw * TW];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int chain = xcd_swizzle(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x));
  const int b = chain / p.n_mblocks;
  const int mb = chain - b * p.n_mblocks;
  const int m0 = mb * MB + lane * V;
  const bool lane_ok = m0 < p.M;
  const int gpw = MB / p.gs;
  const int lpg = p.gs / V;
  const int my_g = lane / lpg;
  const int g_base = mb * gpw;
  const bool reset_first = (p.flags & SPARC_FLAG_RESET_FIRST) != 0;
  const uint32_t lane_bytes = static_cast<uint32_t>(lane * V * ESZ);
  const int64_t row0 = static_cast<int64_t>(b) * p.T;
  const int64_t mbase = static_cast<int64_t>(mb) * MB;
  const int64_t stride = static_cast<int64_t>(p.M) * ESZ;     // bytes per step, [B,T,M]
  const int64_t ostride = (RELU ? 2 : 1) * stride;             // bytes per step of y
  float* tab = s_tab[wave];

  if (wave == 0) {
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int64_t hi = static_cast<int64_t>(b) * p.M + m0 + v;
      s_carry[0][0][v][lane] = (p.h0_re && lane_ok) ? p.h0_re[hi] : 0.0f;
      if constexpr (CPLX) s_carry[0][1][v][lane] = (p.h0_im && lane_ok) ? p.h0_im[hi] : 0.0f;
    }
  }

  RawT wr[2][S], wi[2][S];
  GateBlock<S> gb[2];
  auto load_chunk = [&](int hb, int c) {
    const int t0 = c * C + wave * S;
    const int64_t off = wave_uniform(((row0 + t0) * p.M + mbase) * ESZ);
#pragma unroll
    for (int s = 0; s < S; ++s) {
      if (t0 + s < p.T && lane_ok) {
        wr[hb][s] = ldb<RawT>(p.w_re, off + s * stride, lane_bytes);
        if constexpr (CPLX) wi[hb][s] = ldb<RawT>(p.w_im, off + s * stride, lane_bytes);
      } else {
        float z[V] = {};
        wr[hb][s] = pack<IO, V>(z);
        wi[hb][s] = wr[hb][s];
      }
    }
    load_gate_pairs<TR, IO, S>(p, b, t0, g_base, gpw, lane, gb[hb]);
  };

  load_chunk(0, 0);
  for (int c0 = 0; c0 < p.n_chunks; c0 += 2) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = c0 + h;
      if (c >= p.n_chunks) break;
      const int t0 = c * C + wave * S;
      if (c + 1 < p.n_chunks) load_chunk(1 - h, c + 1);
      fill_tab<TR, IO, S, TW>(p, t0, g_base, gpw, lane, reset_first, gb[h], tab);
      __builtin_amdgcn_wave_barrier();
      float ar[S], ai[S];
#pragma unroll
      for (int s = 0; s < S; ++s) {
        ar[s] = tab[(s * gpw + my_g) * TW];
        ai[s] = CPLX ? tab[(s * gpw + my_g) * TW + 1] : 0.0f;
      }
      // local scan from zero: P (shared by the lane's modes), Q (per mode)
      float Pr = 1.0f, Pi = 0.0f, Qr[V], Qi[V];
#pragma unroll
      for (int v = 0; v < V; ++v) { Qr[v] = 0.0f; Qi[v] = 0.0f; }
#pragma unroll
      for (int s = 0; s < S; ++s) {
        float xr[V], xi[V];
        unpack<IO, V>(wr[h][s], xr);
        if constexpr (CPLX) unpack<IO, V>(wi[h][s], xi);
#pragma unroll
        for (int v = 0; v < V; ++v) {
          if constexpr (CPLX) {
            const float nr = fmaf(ar[s], Qr[v], fmaf(-ai[s], Qi[v], xr[v]));
            const float ni = fmaf(ai[s], Qr[v], fmaf(ar[s], Qi[v], xi[v]));
            Qr[v] = nr;
            Qi[v] = ni;
          } else {
            Qr[v] = fmaf(ar[s], Qr[v], xr[v]);
          }
        }
        if constexpr (CPLX) {
          const float nr = ar[s] * Pr - ai[s] * Pi;
          const float ni = ar[s] * Pi + ai[s] * Pr;
          Pr = nr;
          Pi = ni;
        } else {
          Pr *= ar[s];
        }
      }
      s_p[h][wave][0][lane] = Pr;
      if constexpr (CPLX) s_p[h][wave][1][lane] = Pi;
#pragma unroll
      for (int v = 0; v < V; ++v) {
        s_q[h][wave][0][v][lane] = Qr[v];
        if constexpr (CPLX) s_q[h][wave][1][v][lane] = Qi[v];
      }
      __syncthreads();
      // start state of this wave: maps 0..wave-1 applied to the chunk carry;
      // the last wave also applies its own map: the carry of the next chunk
      float sr[V], si[V], er[V], ei[V];
#pragma unroll
      for (int v = 0; v < V; ++v) {
        sr[v] = s_carry[h][0][v][lane];
        si[v] = CPLX ? s_carry[h][1][v][lane] : 0.0f;
      }
      const int n_maps = (wave == NW - 1) ? NW : wave;
      for (int k = 0; k < n_maps; ++k) {
        if (k == wave) {
#pragma unroll
          for (int v = 0; v < V; ++v) { er[v] = sr[v]; ei[v] = si[v]; }
        }
        const float pr = s_p[h][k][0][lane];
        const float pi = CPLX ? s_p[h][k][1][lane] : 0.0f;
#pragma unroll
        for (int v = 0; v < V; ++v) {
          if constexpr (CPLX) {
            const float nr = fmaf(pr, sr[v], fmaf(-pi, si[v], s_q[h][k][0][v][lane]));
            const float ni = fmaf(pr, si[v], fmaf(pi, sr[v], s_q[h][k][1][v][lane]));
            sr[v] = nr;
            si[v] = ni;
          } else {
            sr[v] = fmaf(pr, sr[v], s_q[h][k][0][v][lane]);
          }
        }
      }
      if (wave == NW - 1) {
#pragma unroll
        for (int v = 0; v < V; ++v) {
          s_carry[1 - h][0][v][lane] = sr[v];
          if constexpr (CPLX) s_carry[1 - h][1][v][lane] = si[v];
        }
        if (lane_ok) {
          float* dst = p.chunk_state + ((static_cast<int64_t>(b) * p.n_chunks + c) * p.M + m0) * NH;
#pragma unroll
          for (int v = 0; v < V; ++v) {
            dst[v * NH] = sr[v];
            if constexpr (CPLX) dst[v * NH + 1] = si[v];
          }
        }
#pragma unroll
        for (int v = 0; v < V; ++v) { sr[v] = er[v]; si[v] = ei[v]; }
      }
      // replay and store
      if (lane_ok) {
        const int64_t yoff = wave_uniform(((row0 + t0) * (RELU ? 2 * p.M : p.M) + mbase) * ESZ);
#pragma unroll
        for (int s = 0; s < S; ++s) {
          float xr[V], xi[V];
          unpack<IO, V>(wr[h][s], xr);
          if constexpr (CPLX) unpack<IO, V>(wi[h][s], xi);
#pragma unroll
          for (int v = 0; v < V; ++v) {
            if constexpr (CPLX) {
              const float nr = fmaf(ar[s], sr[v], fmaf(-ai[s], si[v], xr[v]));
              const float ni = fmaf(ai[s], sr[v], fmaf(ar[s], si[v], xi[v]));
              sr[v] = nr;
              si[v] = ni;
            } else {
              sr[v] = fmaf(ar[s], sr[v], xr[v]);
            }
          }
          if (t0 + s < p.T) {
            const int64_t o = yoff + s * ostride;
            if constexpr (RELU) {
              float rr[V], ri[V];
#pragma unroll
              for (int v = 0; v < V; ++v) { rr[v] = fmaxf(sr[v], 0.0f); ri[v] = fmaxf(si[v], 0.0f); }
              stb<RawT>(p.y_re, o, lane_bytes, pack<IO, V>(rr));
              stb<RawT>(p.y_re, o + stride, lane_bytes, pack<IO, V>(ri));
            } else {
              stb<RawT>(p.y_re, o, lane_bytes, pack<IO, V>(sr));
              if constexpr (CPLX) stb<RawT>(p.y_im, o, lane_bytes, pack<IO, V>(si));
            }
          }
        }
      }
    }
  }
}

template <int TR, typename IO, int V, int S, int NW, bool RELU>
__global__ void __launch_bounds__(NW * 64, 2)
chain_bwd_fast_kernel(ScanArgs p) {
  static_assert(!tr_g32(TR), "lane-shared kernels read gates in the I/O dtype");
  if (blockIdx.x == 0 && threadIdx.x == 0) *p.error = 0u;  // no waits here: never an error
  constexpr bool CPLX = TR != TR_REAL;
  constexpr int C = S * NW;
  constexpr int MB = 64 * V;
  constexpr int NH = CPLX ? 2 : 1;
  constexpr int R = fast_rounds(S);
  constexpr int TW = (TR == TR_POLAR) ? 4 : (CPLX ? 2 : 1);
  constexpr int ESZ = sizeof(IO);
  constexpr int NG = CPLX ? 2 : 1;    // gate gradients per (step, group)
  constexpr int RED = S * NG + 1;     // padded LDS row of one lane's partial gate gradients
  using RawT = typename Raw<IO, V>::T;
  // Forward maps (s_fp, s_fq) and reverse maps (s_rp, s_rq) of every wave's
  // sub-chunk, in two buffers by chunk parity.  Without relu both are built
  // before one barrier and read after it; a wave that runs ahead into the
  // next chunk writes the other buffer, and cannot reach the one after that
  // before every wave has passed the next chunk's barrier.  With relu the
  // reverse map needs the recomputed states, so the reverse maps are built
  // after a first barrier and read after a second.
  __shared__ float s_fp[2][NW][NH][64];
  __shared__ float s_fq[2][NW][NH][V][64];
  __shared__ float s_rp[2][NW][NH][64];
  __shared__ float s_rq[2][NW][NH][V][64];
  __shared__ float s_xi[2][NH][V][64];
  __shared__ float s_tab[NW][S * kFastMaxGpw * TW];
  __shared__ float s_red[NW][64 * RED];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int chain = xcd_swizzle(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x));
  const int b = chain / p.n_mblocks;
  const int mb = chain - b * p.n_mblocks;
  const int m0 = mb * MB + lane * V;
  const bool lane_ok = m0 < p.M;
  const int gpw = MB / p.gs;
  const int lpg = p.gs / V;
  const int my_g = lane / lpg;
  const int g_base = mb * gpw;
  const bool reset_first = (p.flags & SPARC_FLAG_RESET_FIRST) != 0;
  const uint32_t lane_bytes = static_cast<uint32_t>(lane * V * ESZ);
  const int64_t row0 = static_cast<int64_t>(b) * p.T;
  const int64_t mbase = static_cast<int64_t>(mb) * MB;
  const int64_t stride = static_cast<int64_t>(p.M) * ESZ;
  const int64_t dstride = (RELU ? 2 : 1) * stride;  // bytes per step of dy
  float* tab = s_tab[wave];
  float* red = s_red[wave];

  if (wave == 0) {
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int64_t hi = static_cast<int64_t>(b) * p.M + m0 + v;
      s_xi[(p.n_chunks - 1) & 1][0][v][lane] = (p.dlast_re && lane_ok) ? p.dlast_re[hi] : 0.0f;
      if constexpr (CPLX) s_xi[(p.n_chunks - 1) & 1][1][v][lane] = (p.dlast_im && lane_ok) ? p.dlast_im[hi] : 0.0f;
    }
  }

  RawT wr[2][S], wi[2][S], dr[2][S], di[2][S];
  GateBlock<S> gb[2];
  float hs[2][V * NH];
  auto load_chunk = [&](int hb, int c) {
    const int t0 = c * C + wave * S;
    const int64_t off = wave_uniform(((row0 + t0) * p.M + mbase) * ESZ);
    const int64_t doff = wave_uniform(((row0 + t0) * (RELU ? 2 * p.M : p.M) + mbase) * ESZ);
#pragma unroll
    for (int s = 0; s < S; ++s) {
      if (t0 + s < p.T && lane_ok) {
        wr[hb][s] = ldb<RawT>(p.w_re, off + s * stride, lane_bytes);
        if constexpr (CPLX) wi[hb][s] = ldb<RawT>(p.w_im, off + s * stride, lane_bytes);
        if constexpr (RELU) {
          dr[hb][s] = ldb<RawT>(p.dy_re, doff + s * dstride, lane_bytes);
          di[hb][s] = ldb<RawT>(p.dy_re, doff + s * dstride + stride, lane_bytes);
        } else {
          dr[hb][s] = ldb<RawT>(p.dy_re, doff + s * dstride, lane_bytes);
          if constexpr (CPLX) di[hb][s] = ldb<RawT>(p.dy_im, doff + s * dstride, lane_bytes);
        }
      } else {
        float z[V] = {};
        wr[hb][s] = pack<IO, V>(z);
        wi[hb][s] = wr[hb][s];
        dr[hb][s] = wr[hb][s];
        di[hb][s] = wr[hb][s];
      }
    }
    load_gate_pairs<TR, IO, S>(p, b, t0, g_base, gpw, lane, gb[hb]);
#pragma unroll
    for (int v = 0; v < V; ++v) {
      float h_r = 0.0f, h_i = 0.0f;
      if (lane_ok) {
        if (c == 0) {
          const int64_t hi = static_cast<int64_t>(b) * p.M + m0 + v;
          if (p.h0_re) { h_r = p.h0_re[hi]; if constexpr (CPLX) h_i = p.h0_im[hi]; }
        } else {
          const int64_t ci_ = ((static_cast<int64_t>(b) * p.n_chunks + c - 1) * p.M + m0 + v) * NH;
          h_r = p.chunk_state_in[ci_];
          if constexpr (CPLX) h_i = p.chunk_state_in[ci_ + 1];
        }
      }
      hs[hb][v * NH] = h_r;
      if constexpr (CPLX) hs[hb][v * NH + 1] = h_i;
    }
  };

  load_chunk(0, p.n_chunks - 1);
  for (int c0 = p.n_chunks - 1; c0 >= 0; c0 -= 2) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = c0 - h;
      if (c < 0) break;
      const int t0 = c * C + wave * S;
      const int xb = c & 1;  // s_xi buffer holding the adjoint entering this chunk
      if (c - 1 >= 0) load_chunk(1 - h, c - 1);
      const uint32_t rmask = fill_tab<TR, IO, S, TW>(p, t0, g_base, gpw, lane, reset_first, gb[h], tab);
      __builtin_amdgcn_wave_barrier();
      float ar[S], ai[S];
#pragma unroll
      for (int s = 0; s < S; ++s) {
        ar[s] = tab[(s * gpw + my_g) * TW];
        ai[s] = CPLX ? tab[(s * gpw + my_g) * TW + 1] : 0.0f;
      }
      // forward map of the sub-chunk
      {
        float Pr = 1.0f, Pi = 0.0f, Qr[V], Qi[V];
#pragma unroll
        for (int v = 0; v < V; ++v) { Qr[v] = 0.0f; Qi[v] = 0.0f; }
#pragma unroll
        for (int s = 0; s < S; ++s) {
          float xr[V], xi[V];
          unpack<IO, V>(wr[h][s], xr);
          if constexpr (CPLX) unpack<IO, V>(wi[h][s], xi);
#pragma unroll
          for (int v = 0; v < V; ++v) {
            if constexpr (CPLX) {
              const float nr = fmaf(ar[s], Qr[v], fmaf(-ai[s], Qi[v], xr[v]));
              const float ni = fmaf(ai[s], Qr[v], fmaf(ar[s], Qi[v], xi[v]));
              Qr[v] = nr;
              Qi[v] = ni;
            } else {
              Qr[v] = fmaf(ar[s], Qr[v], xr[v]);
            }
          }
          if constexpr (CPLX) {
            const float nr = ar[s] * Pr - ai[s] * Pi;
            const float ni = ar[s] * Pi + ai[s] * Pr;
            Pr = nr;
            Pi = ni;
          } else {
            Pr *= ar[s];
          }
        }
        s_fp[xb][wave][0][lane] = Pr;
        s_rp[xb][wave][0][lane] = Pr;   // the reverse product is the conjugate
        if constexpr (CPLX) { s_fp[xb][wave][1][lane] = Pi; s_rp[xb][wave][1][lane] = -Pi; }
#pragma unroll
        for (int v = 0; v < V; ++v) {
          s_fq[xb][wave][0][v][lane] = Qr[v];
          if constexpr (CPLX) s_fq[xb][wave][1][v][lane] = Qi[v];
        }
      }
      // output gradient of step s; with relu masked by the state after step s
      auto dy_raw = [&](int s, float (&gy_r)[V], float (&gy_i)[V]) {
        unpack<IO, V>(dr[h][s], gy_r);
        if constexpr (CPLX) unpack<IO, V>(di[h][s], gy_i);
        else {
#pragma unroll
          for (int v = 0; v < V; ++v) gy_i[v] = 0.0f;
        }
      };
      // reverse map of the sub-chunk from zero: xi_out = conj(prod a) xi_in + Q
      auto reverse_map = [&](const float (&hpr)[S + 1][V], const float (&hpi)[S + 1][V]) {
        float Xr[V], Xi[V];
#pragma unroll
        for (int v = 0; v < V; ++v) { Xr[v] = 0.0f; Xi[v] = 0.0f; }
#pragma unroll
        for (int s = S - 1; s >= 0; --s) {
          float gy_r[V], gy_i[V];
          dy_raw(s, gy_r, gy_i);
#pragma unroll
          for (int v = 0; v < V; ++v) {
            if constexpr (RELU) {
              gy_r[v] = hpr[s + 1][v] > 0.0f ? gy_r[v] : 0.0f;
              gy_i[v] = hpi[s + 1][v] > 0.0f ? gy_i[v] : 0.0f;
            }
            const float lr = gy_r[v] + Xr[v];
            const float li = gy_i[v] + Xi[v];
            if constexpr (CPLX) {
              Xr[v] = fmaf(ar[s], lr, ai[s] * li);
              Xi[v] = fmaf(ar[s], li, -ai[s] * lr);
            } else {
              Xr[v] = ar[s] * lr;
            }
          }
        }
#pragma unroll
        for (int v = 0; v < V; ++v) {
          s_rq[xb][wave][0][v][lane] = Xr[v];
          if constexpr (CPLX) s_rq[xb][wave][1][v][lane] = Xi[v];
        }
      };
      // start state of this wave: forward maps 0..wave-1 applied to the chunk start
      auto start_state = [&](float (&hr)[V], float (&hi)[V]) {
#pragma unroll
        for (int v = 0; v < V; ++v) { hr[v] = hs[h][v * NH]; hi[v] = CPLX ? hs[h][v * NH + 1] : 0.0f; }
        for (int k = 0; k < wave; ++k) {
          const float pr = s_fp[xb][k][0][lane];
          const float pi = CPLX ? s_fp[xb][k][1][lane] : 0.0f;
#pragma unroll
          for (int v = 0; v < V; ++v) {
            if constexpr (CPLX) {
              const float nr = fmaf(pr, hr[v], fmaf(-pi, hi[v], s_fq[xb][k][0][v][lane]));
              const float ni = fmaf(pr, hi[v], fmaf(pi, hr[v], s_fq[xb][k][1][v][lane]));
              hr[v] = nr;
              hi[v] = ni;
            } else {
              hr[v] = fmaf(pr, hr[v], s_fq[xb][k][0][v][lane]);
            }
          }
        }
      };
      // recompute the state before every step (and after the last one)
      auto recompute = [&](float (&hr)[V], float (&hi)[V], float (&hpr)[S + 1][V], float (&hpi)[S + 1][V]) {
#pragma unroll
        for (int s = 0; s < S; ++s) {
          float xr[V], xi[V];
          unpack<IO, V>(wr[h][s], xr);
          if constexpr (CPLX) unpack<IO, V>(wi[h][s], xi);
#pragma unroll
          for (int v = 0; v < V; ++v) {
            hpr[s][v] = hr[v];
            hpi[s][v] = CPLX ? hi[v] : 0.0f;
            if constexpr (CPLX) {
              const float nr = fmaf(ar[s], hr[v], fmaf(-ai[s], hi[v], xr[v]));
              const float ni = fmaf(ai[s], hr[v], fmaf(ar[s], hi[v], xi[v]));
              hr[v] = nr;
              hi[v] = ni;
            } else {
              hr[v] = fmaf(ar[s], hr[v], xr[v]);
            }
          }
        }
#pragma unroll
        for (int v = 0; v < V; ++v) { hpr[S][v] = hr[v]; hpi[S][v] = CPLX ? hi[v] : 0.0f; }
      };

      float hpr[S + 1][V], hpi[S + 1][V];
      float hr[V], hi[V];
      if constexpr (!RELU) {
        reverse_map(hpr, hpi);  // (states unused without relu)
        __syncthreads();        // maps of all waves visible
        start_state(hr, hi);
        recompute(hr, hi, hpr, hpi);
      } else {
        __syncthreads();        // B1: forward maps
        start_state(hr, hi);
        recompute(hr, hi, hpr, hpi);
        reverse_map(hpr, hpi);
        __syncthreads();        // B2: reverse maps
      }
      // adjoint entering this wave: reverse maps NW-1 .. wave+1 applied to the chunk's
      float xr[V], xi[V], er[V], ei[V];
#pragma unroll
      for (int v = 0; v < V; ++v) {
        xr[v] = s_xi[xb][0][v][lane];
        xi[v] = CPLX ? s_xi[xb][1][v][lane] : 0.0f;
      }
      const int k_end = (wave == 0) ? -1 : wave;   // wave 0 also applies map 0 -> next carry
      for (int k = NW - 1; k > k_end; --k) {
        if (k == wave) {
#pragma unroll
          for (int v = 0; v < V; ++v) { er[v] = xr[v]; ei[v] = xi[v]; }
        }
        const float pr = s_rp[xb][k][0][lane];
        const float pi = CPLX ? s_rp[xb][k][1][lane] : 0.0f;
#pragma unroll
        for (int v = 0; v < V; ++v) {
          if constexpr (CPLX) {
            const float nr = fmaf(pr, xr[v], fmaf(-pi, xi[v], s_rq[xb][k][0][v][lane]));
            const float ni = fmaf(pr, xi[v], fmaf(pi, xr[v], s_rq[xb][k][1][v][lane]));
            xr[v] = nr;
            xi[v] = ni;
          } else {
            xr[v] = fmaf(pr, xr[v], s_rq[xb][k][0][v][lane]);
          }
        }
      }
      if (wave == 0) {
        if (c > 0) {
#pragma unroll
          for (int v = 0; v < V; ++v) {
            s_xi[1 - xb][0][v][lane] = xr[v];
            if constexpr (CPLX) s_xi[1 - xb][1][v][lane] = xi[v];
          }
        } else if (lane_ok && p.dh0_re) {
#pragma unroll
          for (int v = 0; v < V; ++v) {
            const int64_t hi2 = static_cast<int64_t>(b) * p.M + m0 + v;
            p.dh0_re[hi2] = xr[v];
            if constexpr (CPLX) p.dh0_im[hi2] = xi[v];
          }
        }
#pragma unroll
        for (int v = 0; v < V; ++v) { xr[v] = er[v]; xi[v] = ei[v]; }
      }
      // final reverse pass: dw, and every lane's partial transition gradients
      const int64_t off = wave_uniform(((row0 + t0) * p.M + mbase) * ESZ);
      float d0[S], d1[S];
#pragma unroll
      for (int s = S - 1; s >= 0; --s) {
        float gy_r[V], gy_i[V], lr[V], li[V];
        dy_raw(s, gy_r, gy_i);
#pragma unroll
        for (int v = 0; v < V; ++v) {
          if constexpr (RELU) {
            gy_r[v] = hpr[s + 1][v] > 0.0f ? gy_r[v] : 0.0f;
            gy_i[v] = hpi[s + 1][v] > 0.0f ? gy_i[v] : 0.0f;
          }
          lr[v] = gy_r[v] + xr[v];
          li[v] = gy_i[v] + xi[v];
        }
        if (lane_ok && t0 + s < p.T) {
          stb<RawT>(p.dw_re, off + s * stride, lane_bytes, pack<IO, V>(lr));
          if constexpr (CPLX) stb<RawT>(p.dw_im, off + s * stride, lane_bytes, pack<IO, V>(li));
        }
        float e0 = 0.0f, e1 = 0.0f;
        float cp = 1.0f, sp = 0.0f;
        if constexpr (TR == TR_POLAR) {
          cp = tab[(s * gpw + my_g) * TW + 2];
          sp = tab[(s * gpw + my_g) * TW + 3];
        }
#pragma unroll
        for (int v = 0; v < V; ++v) {
          if constexpr (CPLX) {
            const float gar = fmaf(lr[v], hpr[s][v], li[v] * hpi[s][v]);
            const float gai = fmaf(li[v], hpr[s][v], -lr[v] * hpi[s][v]);
            if constexpr (TR == TR_POLAR) {
              e0 += fmaf(gar, cp, gai * sp);
              e1 += fmaf(gai, ar[s], -gar * ai[s]);
            } else {
              e0 += gar;
              e1 += gai;
            }
            const float nr = fmaf(ar[s], lr[v], ai[s] * li[v]);
            const float ni = fmaf(ar[s], li[v], -ai[s] * lr[v]);
            xr[v] = nr;
            xi[v] = ni;
          } else {
            e0 = fmaf(lr[v], hpr[s][v], e0);
            xr[v] = ar[s] * lr[v];
          }
        }
        d0[s] = e0;
        d1[s] = e1;
      }
      // sum the partials of each (step, group) over the group's lanes through
      // a transpose in LDS; lane l then owns pair l (step l / gpw, group l % gpw)
#pragma unroll
      for (int s = 0; s < S; ++s) {
        red[lane * RED + s * NG] = d0[s];
        if constexpr (CPLX) red[lane * RED + s * NG + 1] = d1[s];
      }
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int idx = r * 64 + lane;
        if (idx < S * gpw) {
          const int step = idx / gpw;
          const int g = idx - step * gpw;
          float a0 = 0.0f, a1 = 0.0f;
          for (int j = 0; j < lpg; ++j) {
            const float* src = red + (g * lpg + j) * RED + step * NG;
            a0 += src[0];
            if constexpr (CPLX) a1 += src[1];
          }
          const int t = t0 + step;
          if (t < p.T && g_base + g < p.G) {  // the last mode block may hold fewer groups
            // a reset step's transition is the constant 0: no gradient
            const bool reset = (rmask >> r) & 1u;
            const int64_t gi = (row0 + t) * p.G + g_base + g;
            store1<IO>(p.dg0, gi, reset ? 0.0f : a0);
            if constexpr (CPLX) store1<IO>(p.dg1, gi, reset ? 0.0f : a1);
          }
        }
      }
    }
  }
}

// Backward that reads the states from the saved forward output y (no relu
// epilogue: y = h rounded to the I/O dtype), as the reference's backward
// does from its saved out_r/out_i (sparc-kernal/backward/scan.py:1325-1329),
// instead of recomputing them from w and the chunk states.  Per chunk: the
// local reverse map of each wave's sub-chunk, one barrier, the composition of
// the later sub-chunks' maps, and the final reverse pass (dw and the gate
// gradients, which take h_{t-1} from row t-1 of y, or from h0 at t = 0).
// Maps are double-buffered by chunk parity, so one barrier per chunk suffices.
template <int TR, typename IO, int V, int S, int NW>
__global__ void __launch_bounds__(NW * 64, 2)
chain_bwd_saved_kernel(ScanArgs p) {
  static_assert(!tr_g32(TR), "lane-shared kernels read gates in the I/O dtype");
  if (blockIdx.x == 0 && threadIdx.x == 0) *p.error = 0u;  // no waits here: never an error
  constexpr bool CPLX = TR != TR_REAL;
  constexpr int C = S * NW;
  constexpr int MB = 64 * V;
  constexpr int NH = CPLX ? 2 : 1;
  constexpr int R = fast_rounds(S);
  constexpr int TW = (TR == TR_POLAR) ? 4 : (CPLX ? 2 : 1);
  constexpr int ESZ = sizeof(IO);
  constexpr int NG = CPLX ? 2 : 1;    // gate gradients per (step, group)
  constexpr int RED = S * NG + 1;     // padded LDS row of one lane's partial gate gradients
  using RawT = typename Raw<IO, V>::T;
  __shared__ float s_rp[2][NW][NH][64];
  __shared__ float s_rq[2][NW][NH][V][64];
  __shared__ float s_xi[2][NH][V][64];
  __shared__ float s_tab[NW][S * kFastMaxGpw * TW];
  __shared__ float s_red[NW][64 * RED];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int chain = xcd_swizzle(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x));
  const int b = chain / p.n_mblocks;
  const int mb = chain - b * p.n_mblocks;
  const int m0 = mb * MB + lane * V;
  const bool lane_ok = m0 < p.M;
  const bool block_full = (mb + 1) * MB <= p.M;  // wave-uniform
  const int gpw = MB / p.gs;
  const int lpg = p.gs / V;
  const int my_g = lane / lpg;
  const int g_base = mb * gpw;
  const bool reset_first = (p.flags & SPARC_FLAG_RESET_FIRST) != 0;
  const uint32_t lane_bytes = static_cast<uint32_t>(lane * V * ESZ);
  const int64_t row0 = static_cast<int64_t>(b) * p.T;
  const int64_t mbase = static_cast<int64_t>(mb) * MB;
  const int64_t stride = static_cast<int64_t>(p.M) * ESZ;
  float* tab = s_tab[wave];
  float* red = s_red[wave];

  if (wave == 0) {
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int64_t hi = static_cast<int64_t>(b) * p.M + m0 + v;
      s_xi[(p.n_chunks - 1) & 1][0][v][lane] = (p.dlast_re && lane_ok) ? p.dlast_re[hi] : 0.0f;
      if constexpr (CPLX) s_xi[(p.n_chunks - 1) & 1][1][v][lane] = (p.dlast_im && lane_ok) ? p.dlast_im[hi] : 0.0f;
    }
  }

  // dy rows t0 .. t0+S-1 and y rows t0-1 .. t0+S-2 (the state before each step)
  RawT dr[2][S], di[2][S], yr[2][S], yi[2][S];
  GateBlock<S> gb[2];
  auto load_chunk = [&](int hb, int c) {
    const int t0 = c * C + wave * S;
    const int64_t off = wave_uniform(((row0 + t0) * p.M + mbase) * ESZ);
    if (block_full && t0 > 0 && t0 + S <= p.T) {
#pragma unroll
      for (int s = 0; s < S; ++s) {
        dr[hb][s] = ldb<RawT>(p.dy_re, off + s * stride, lane_bytes);
        yr[hb][s] = ldb<RawT>(p.y_re, off + (s - 1) * stride, lane_bytes);
        if constexpr (CPLX) {
          di[hb][s] = ldb<RawT>(p.dy_im, off + s * stride, lane_bytes);
          yi[hb][s] = ldb<RawT>(p.y_im, off + (s - 1) * stride, lane_bytes);
        }
      }
    } else {
      float z[V] = {};
      const RawT zero = pack<IO, V>(z);
#pragma unroll
      for (int s = 0; s < S; ++s) {
        const int t = t0 + s;
        dr[hb][s] = zero; di[hb][s] = zero; yr[hb][s] = zero; yi[hb][s] = zero;
        if (lane_ok && t < p.T) {
          dr[hb][s] = ldb<RawT>(p.dy_re, off + s * stride, lane_bytes);
          if constexpr (CPLX) di[hb][s] = ldb<RawT>(p.dy_im, off + s * stride, lane_bytes);
          if (t > 0) {
            yr[hb][s] = ldb<RawT>(p.y_re, off + (s - 1) * stride, lane_bytes);
            if constexpr (CPLX) yi[hb][s] = ldb<RawT>(p.y_im, off + (s - 1) * stride, lane_bytes);
          }
        }
      }
    }
    load_gate_pairs<TR, IO, S>(p, b, t0, g_base, gpw, lane, gb[hb]);
  };

  load_chunk(0, p.n_chunks - 1);
  for (int c0 = p.n_chunks - 1; c0 >= 0; c0 -= 2) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = c0 - h;
      if (c < 0) break;
      const int t0 = c * C + wave * S;
      const int xb = c & 1;  // buffers of this chunk (maps, entering adjoint)
      if (c - 1 >= 0) load_chunk(1 - h, c - 1);
      const uint32_t rmask = fill_tab<TR, IO, S, TW>(p, t0, g_base, gpw, lane, reset_first, gb[h], tab);
      __builtin_amdgcn_wave_barrier();
      float ar[S], ai[S];
#pragma unroll
      for (int s = 0; s < S; ++s) {
        ar[s] = tab[(s * gpw + my_g) * TW];
        ai[s] = CPLX ? tab[(s * gpw + my_g) * TW + 1] : 0.0f;
      }
      // reverse map of the sub-chunk from zero: xi_out = conj(prod a) xi_in + X
      {
        float Xr[V], Xi[V], Pr = 1.0f, Pi = 0.0f;
#pragma unroll
        for (int v = 0; v < V; ++v) { Xr[v] = 0.0f; Xi[v] = 0.0f; }
#pragma unroll
        for (int s = S - 1; s >= 0; --s) {
          float gy_r[V], gy_i[V];
          unpack<IO, V>(dr[h][s], gy_r);
          if constexpr (CPLX) unpack<IO, V>(di[h][s], gy_i);
#pragma unroll
          for (int v = 0; v < V; ++v) {
            if constexpr (CPLX) {
              const float lr = gy_r[v] + Xr[v];
              const float li = gy_i[v] + Xi[v];
              Xr[v] = fmaf(ar[s], lr, ai[s] * li);
              Xi[v] = fmaf(ar[s], li, -ai[s] * lr);
            } else {
              Xr[v] = ar[s] * (gy_r[v] + Xr[v]);
            }
          }
          if constexpr (CPLX) {
            const float nr = ar[s] * Pr - ai[s] * Pi;
            const float ni = ar[s] * Pi + ai[s] * Pr;
            Pr = nr;
            Pi = ni;
          } else {
            Pr *= ar[s];
          }
        }
        s_rp[xb][wave][0][lane] = Pr;
        if constexpr (CPLX) s_rp[xb][wave][1][lane] = -Pi;
#pragma unroll
        for (int v = 0; v < V; ++v) {
          s_rq[xb][wave][0][v][lane] = Xr[v];
          if constexpr (CPLX) s_rq[xb][wave][1][v][lane] = Xi[v];
        }
      }
      __syncthreads();  // reverse maps of all waves visible
      // adjoint entering this wave: maps NW-1 .. wave+1 applied to the chunk's
      float xr[V], xi[V], er[V], ei[V];
#pragma unroll
      for (int v = 0; v < V; ++v) {
        xr[v] = s_xi[xb][0][v][lane];
        xi[v] = CPLX ? s_xi[xb][1][v][lane] : 0.0f;
      }
      const int k_end = (wave == 0) ? -1 : wave;   // wave 0 also applies map 0 -> next carry
      for (int k = NW - 1; k > k_end; --k) {
        if (k == wave) {
#pragma unroll
          for (int v = 0; v < V; ++v) { er[v] = xr[v]; ei[v] = xi[v]; }
        }
        const float pr = s_rp[xb][k][0][lane];
        const float pi = CPLX ? s_rp[xb][k][1][lane] : 0.0f;
#pragma unroll
        for (int v = 0; v < V; ++v) {
          if constexpr (CPLX) {
            const float nr = fmaf(pr, xr[v], fmaf(-pi, xi[v], s_rq[xb][k][0][v][lane]));
            const float ni = fmaf(pr, xi[v], fmaf(pi, xr[v], s_rq[xb][k][1][v][lane]));
            xr[v] = nr;
            xi[v] = ni;
          } else {
            xr[v] = fmaf(pr, xr[v], s_rq[xb][k][0][v][lane]);
          }
        }
      }
      if (wave == 0) {
        if (c > 0) {
#pragma unroll
          for (int v = 0; v < V; ++v) {
            s_xi[1 - xb][0][v][lane] = xr[v];
            if constexpr (CPLX) s_xi[1 - xb][1][v][lane] = xi[v];
          }
        } else if (lane_ok && p.dh0_re) {
#pragma unroll
          for (int v = 0; v < V; ++v) {
            const int64_t hi2 = static_cast<int64_t>(b) * p.M + m0 + v;
            p.dh0_re[hi2] = xr[v];
            if constexpr (CPLX) p.dh0_im[hi2] = xi[v];
          }
        }
        // wave 0's own entering adjoint, saved before it applied map 0
#pragma unroll
        for (int v = 0; v < V; ++v) { xr[v] = er[v]; xi[v] = ei[v]; }
      }
      // final reverse pass: dw, and every lane's partial transition gradients
      const int64_t off = wave_uniform(((row0 + t0) * p.M + mbase) * ESZ);
#pragma unroll
      for (int s = S - 1; s >= 0; --s) {
        float gy_r[V], gy_i[V], lr[V], li[V], hr[V], hi[V];
        unpack<IO, V>(dr[h][s], gy_r);
        unpack<IO, V>(yr[h][s], hr);
        if constexpr (CPLX) {
          unpack<IO, V>(di[h][s], gy_i);
          unpack<IO, V>(yi[h][s], hi);
        }
        if (t0 + s == 0) {  // the state before step 0 is h0 (fp32), or zero
#pragma unroll
          for (int v = 0; v < V; ++v) {
            const int64_t i0 = static_cast<int64_t>(b) * p.M + m0 + v;
            hr[v] = (p.h0_re && lane_ok) ? p.h0_re[i0] : 0.0f;
            if constexpr (CPLX) hi[v] = (p.h0_im && lane_ok) ? p.h0_im[i0] : 0.0f;
          }
        }
#pragma unroll
        for (int v = 0; v < V; ++v) {
          lr[v] = gy_r[v] + xr[v];
          if constexpr (CPLX) li[v] = gy_i[v] + xi[v];
        }
        if (lane_ok && t0 + s < p.T) {
          stb<RawT>(p.dw_re, off + s * stride, lane_bytes, pack<IO, V>(lr));
          if constexpr (CPLX) stb<RawT>(p.dw_im, off + s * stride, lane_bytes, pack<IO, V>(li));
        }
        float e0 = 0.0f, e1 = 0.0f;
        float cp = 1.0f, sp = 0.0f;
        if constexpr (TR == TR_POLAR) {
          cp = tab[(s * gpw + my_g) * TW + 2];
          sp = tab[(s * gpw + my_g) * TW + 3];
        }
#pragma unroll
        for (int v = 0; v < V; ++v) {
          if constexpr (CPLX) {
            const float gar = fmaf(lr[v], hr[v], li[v] * hi[v]);
            const float gai = fmaf(li[v], hr[v], -lr[v] * hi[v]);
            if constexpr (TR == TR_POLAR) {
              e0 += fmaf(gar, cp, gai * sp);
              e1 += fmaf(gai, ar[s], -gar * ai[s]);
            } else {
              e0 += gar;
              e1 += gai;
            }
            xr[v] = fmaf(ar[s], lr[v], ai[s] * li[v]);
            xi[v] = fmaf(ar[s], li[v], -ai[s] * lr[v]);
          } else {
            e0 = fmaf(lr[v], hr[v], e0);
            xr[v] = ar[s] * lr[v];
          }
        }
        red[lane * RED + s * NG] = e0;
        if constexpr (CPLX) red[lane * RED + s * NG + 1] = e1;
      }
      // sum the partials of each (step, group) over the group's lanes through
      // a transpose in LDS; lane l then owns pair l (step l / gpw, group l % gpw)
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int idx = r * 64 + lane;
        if (idx < S * gpw) {
          const int step = idx / gpw;
          const int g = idx - step * gpw;
          float a0 = 0.0f, a1 = 0.0f;
          for (int j = 0; j < lpg; ++j) {
            const float* src = red + (g * lpg + j) * RED + step * NG;
            a0 += src[0];
            if constexpr (CPLX) a1 += src[1];
          }
          const int t = t0 + step;
          if (t < p.T && g_base + g < p.G) {  // the last mode block may hold fewer groups
            // a reset step's transition is the constant 0: no gradient
            const bool reset = (rmask >> r) & 1u;
            const int64_t gi = (row0 + t) * p.G + g_base + g;
            store1<IO>(p.dg0, gi, reset ? 0.0f : a0);
            if constexpr (CPLX) store1<IO>(p.dg1, gi, reset ? 0.0f : a1);
          }
        }
      }
      __builtin_amdgcn_wave_barrier();
    }
  }
}

// ---------------------------------------------------------------------------
// Serial kernels for lane-shared gates: one chain (batch row, block of 64*V
// modes) per workgroup of two waves.
//   * Wave 0 streams the chain.  It walks every step in order (forward) or in
//     reverse (backward, reading the states from the saved output), one
//     complex multiply-add per mode and step, and loads the next block of S
//     steps of the planes into registers while it computes the current one.
//   * Wave 1 does the rest.  It loads the gates two blocks ahead and turns
//     them into the transition table of the next block (double-buffered in
//     LDS).  Backward, it also sums the transition gradients of the previous
//     block over the lanes of each group (an LDS transpose) and stores the
//     gate gradients.
// Wave 0 thus issues no memory instruction but its plane loads and stores, so
// the wait before a block covers that block's loads only, never the prefetch
// of the next one (a gate load in the same wave, used one block later, made
// the compiler drain the whole prefetch).  One workgroup barrier per block
// hands the buffers over.  Parallelism is over chains only; the plan picks
// these kernels when there are enough chains to fill the GPU.
// ---------------------------------------------------------------------------
constexpr int kStateChunk = 64;  // steps per saved chunk state

// blocks of gates in flight in the helper wave (loaded kGateDepth-1 blocks
// before their table is built); an even number
#ifndef SPARC_GATE_DEPTH
#define SPARC_GATE_DEPTH 4
#endif
constexpr int kGateDepth = SPARC_GATE_DEPTH;
// At least 4: a block's gates are loaded kGateDepth-1 blocks ahead and its
// table is built from them one block ahead, so the load must come at least two
// iterations before the build (the loops issue an iteration's load after its
// build).
static_assert(kGateDepth % 2 == 0 && kGateDepth >= 4, "the loops pair plane buffers with even depths, 4 or more");
#ifndef SPARC_SERIAL_SWIZZLE
#define SPARC_SERIAL_SWIZZLE 1
#endif

// A serial workgroup's chain and steps: segment seg_lo + blockIdx / n_chains
// of t_seg steps with time segments, else the whole sequence.
struct SerialPos {
  int b, mb, seg, t_begin, t_end;
};
__device__ __forceinline__ SerialPos serial_pos(const ScanArgs& p) {
  const int idx = SPARC_SERIAL_SWIZZLE ? xcd_swizzle(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x))
                                       : static_cast<int>(blockIdx.x);
  const int sj = idx / p.n_chains, chain = idx - sj * p.n_chains;
  SerialPos c;
  c.b = chain / p.n_mblocks;
  c.mb = chain - c.b * p.n_mblocks;
  const bool segs = p.n_seg > 1;
  c.seg = segs ? p.seg_lo + sj : 0;
  c.t_begin = segs ? c.seg * p.t_seg : 0;
  c.t_end = segs ? min(p.T, c.t_begin + p.t_seg) : p.T;
  return c;
}

// SUMMARY (time segments): the segment's map from a zero state, h_out = P h_in
// + Q, into seg_sum; no stores of y or of the chunk states.  Otherwise the
// segment starts from its entering state in seg_state (h0 for the first
// segment is folded in there by the carry kernel).
template <int TR, typename IO, int V, int S, bool RELU, bool SUMMARY = false>
__global__ void __launch_bounds__(128, 1)
chain_fwd_serial_kernel(ScanArgs p) {
  static_assert(!tr_g32(TR), "lane-shared kernels read gates in the I/O dtype");
  static_assert(kStateChunk % S == 0, "blocks must tile the saved-state chunks");
  if (blockIdx.x == 0 && threadIdx.x == 0) *p.error = 0u;  // no waits here: never an error
  constexpr bool CPLX = TR != TR_REAL;
  constexpr int MB = 64 * V;
  constexpr int NH = CPLX ? 2 : 1;
  constexpr int TW = CPLX ? 2 : 1;
  constexpr int ESZ = sizeof(IO);
  using RawT = typename Raw<IO, V>::T;
  __shared__ float tab[2][S * kFastMaxGpw * TW];

  const SerialPos cp = serial_pos(p);
  const int n_blocks = (cp.t_end - cp.t_begin + S - 1) / S;
  if (n_blocks <= 0) return;  // the whole workgroup: no barrier is skipped by one wave only
  const int lane = threadIdx.x & 63;
  const bool streamer = threadIdx.x < 64;  // wave-uniform
  const int b = cp.b, mb = cp.mb, t_begin = cp.t_begin;
  const int m0 = mb * MB + lane * V;
  const bool lane_ok = m0 < p.M;
  const int gpw = MB / p.gs;
  const int lpg = p.gs / V;
  const int my_g = lane / lpg;
  const int g_base = mb * gpw;
  const bool reset_first = (p.flags & SPARC_FLAG_RESET_FIRST) != 0;
  const uint32_t lane_bytes = static_cast<uint32_t>(lane * V * ESZ);
  const int64_t row0 = static_cast<int64_t>(b) * p.T;
  const int64_t mbase = static_cast<int64_t>(mb) * MB;
  const int64_t stride = static_cast<int64_t>(p.M) * ESZ;   // bytes per step of w
  const int64_t ostride = (RELU ? 2 : 1) * stride;          // bytes per step of y

  float hr[V], hi[V];
  float Pr[V], Pi[V];  // SUMMARY: the product of the segment's transitions
  const bool from_seg = !SUMMARY && p.n_seg > 1;
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int64_t i0 = static_cast<int64_t>(b) * p.M + m0 + v;
    const int64_t si = ((static_cast<int64_t>(b) * p.n_seg + cp.seg) * p.M + m0 + v) * 2;
    if (SUMMARY) {
      hr[v] = 0.0f;
      hi[v] = 0.0f;
    } else if (from_seg) {
      hr[v] = (streamer && lane_ok) ? p.seg_state[si] : 0.0f;
      hi[v] = (streamer && CPLX && lane_ok) ? p.seg_state[si + 1] : 0.0f;
    } else {
      hr[v] = (streamer && p.h0_re && lane_ok) ? p.h0_re[i0] : 0.0f;
      hi[v] = (streamer && CPLX && p.h0_im && lane_ok) ? p.h0_im[i0] : 0.0f;
    }
    Pr[v] = 1.0f;
    Pi[v] = 0.0f;
  }
  // The initial state is loop-carried: complete its loads here, or the
  // compiler, unsure at the loop head whether they are still pending, waits
  // for the whole prefetch before each block.
  wait_vm_all();

  RawT wr[2][S], wi[2][S];     // wave 0: plane registers, double-buffered
  GateBlock<S> gb[kGateDepth];  // wave 1: raw gates of block j in gb[j % kGateDepth]
  // The loads are unconditional: steps past T re-read row T-1 and lanes past
  // M read the first element of their mode block; run_block discards both.
  // (Loads under a branch made the compiler's wait bookkeeping drain the whole
  // prefetch before every block.)
  const uint32_t lane_ld = lane_ok ? lane_bytes : 0u;
  auto load_block = [&](int hb, int k) {
    const int t0 = t_begin + k * S;
    const int64_t off = wave_uniform(((row0 + t0) * p.M + mbase) * ESZ);
    const int last = p.T - 1 - t0;  // the block's last step inside T (wave-uniform)
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int64_t o = off + static_cast<int64_t>(s <= last ? s : last) * stride;
      wr[hb][s] = ldn<RawT, (SPARC_FWD_NT & 1) != 0>(p.w_re, o, lane_ld);
      if constexpr (CPLX) wi[hb][s] = ldn<RawT, (SPARC_FWD_NT & 1) != 0>(p.w_im, o, lane_ld);
    }
  };

  // S steps of one block from transition table tb (identity past T)
  auto run_block = [&](int h, int t0, const float* tb) {
    const bool tail = t0 + S > p.T;  // wave-uniform
    float ar[S], ai[S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
      ar[s] = tb[(s * gpw + my_g) * TW];
      ai[s] = CPLX ? tb[(s * gpw + my_g) * TW + 1] : 0.0f;
    }
    const int64_t yoff = wave_uniform(((row0 + t0) * (RELU ? 2 * p.M : p.M) + mbase) * ESZ);
#pragma unroll
    for (int s = 0; s < S; ++s) {
      float xr[V], xi[V];
      unpack<IO, V>(wr[h][s], xr);
      if constexpr (CPLX) unpack<IO, V>(wi[h][s], xi);
      if (tail && t0 + s >= p.T) {  // no write past T
#pragma unroll
        for (int v = 0; v < V; ++v) { xr[v] = 0.0f; xi[v] = 0.0f; }
      }
#pragma unroll
      for (int v = 0; v < V; ++v) {
        if constexpr (CPLX) {
          const float nr = fmaf(ar[s], hr[v], fmaf(-ai[s], hi[v], xr[v]));
          const float ni = fmaf(ai[s], hr[v], fmaf(ar[s], hi[v], xi[v]));
          hr[v] = nr;
          hi[v] = ni;
          if constexpr (SUMMARY) {  // P <- a P (the identity past T)
            const float pr = fmaf(ar[s], Pr[v], -ai[s] * Pi[v]);
            Pi[v] = fmaf(ai[s], Pr[v], ar[s] * Pi[v]);
            Pr[v] = pr;
          }
        } else {
          hr[v] = fmaf(ar[s], hr[v], xr[v]);
          if constexpr (SUMMARY) Pr[v] *= ar[s];
        }
      }
      if constexpr (SUMMARY) continue;
      if (lane_ok && t0 + s < p.T) {
        const int64_t o = yoff + s * ostride;
        if constexpr (RELU) {
          float rr[V], ri[V];
#pragma unroll
          for (int v = 0; v < V; ++v) { rr[v] = fmaxf(hr[v], 0.0f); ri[v] = fmaxf(hi[v], 0.0f); }
          stn<RawT, (SPARC_FWD_NT & 2) != 0>(p.y_re, o, lane_bytes, pack<IO, V>(rr));
          stn<RawT, (SPARC_FWD_NT & 2) != 0>(p.y_re, o + stride, lane_bytes, pack<IO, V>(ri));
        } else {
          stn<RawT, (SPARC_FWD_NT & 2) != 0>(p.y_re, o, lane_bytes, pack<IO, V>(hr));
          if constexpr (CPLX) stn<RawT, (SPARC_FWD_NT & 2) != 0>(p.y_im, o, lane_bytes, pack<IO, V>(hi));
        }
      }
    }
  };

  if (streamer) {
    load_block(0, 0);
  } else {
#pragma unroll
    for (int d = 0; d < kGateDepth - 1; ++d)
      if (d < n_blocks) load_gate_pairs<TR, IO, S>(p, b, t_begin + d * S, g_base, gpw, lane, gb[d]);
    fill_tab<TR, IO, S, TW>(p, t_begin, g_base, gpw, lane, reset_first, gb[0], tab[0]);
  }
  __syncthreads();
  // block k = k0 + h: planes and table in buffers k & 1 = h & 1, gates in
  // gb[k % kGateDepth] = gb[h] (k0 is a multiple of kGateDepth)
  for (int k0 = 0; k0 < n_blocks; k0 += kGateDepth) {
#pragma unroll
    for (int h = 0; h < kGateDepth; ++h) {
      const int k = k0 + h;
      if (k >= n_blocks) break;
      const int t0 = t_begin + k * S;
      const int x = h & 1;
      if (streamer) {
        // unconditional (the last block re-reads itself): a path without the
        // prefetch would make the waits below cover it as well
        load_block(1 - x, k + 1 < n_blocks ? k + 1 : k);
        run_block(x, t0, tab[x]);
        // the state after the last step of a saved-state chunk (steps past T
        // are the identity, so the last block ends on the state after T-1)
        const int t_end = t0 + S;
        if (!SUMMARY && lane_ok && (t_end % kStateChunk == 0 || t_end >= p.T)) {
          const int c = (min(t_end, p.T) - 1) / kStateChunk;
          float* dst = p.chunk_state + ((static_cast<int64_t>(b) * p.n_chunks + c) * p.M + m0) * NH;
#pragma unroll
          for (int v = 0; v < V; ++v) {
            dst[v * NH] = hr[v];
            if constexpr (CPLX) dst[v * NH + 1] = hi[v];
          }
        }
      } else if (k + 1 < n_blocks) {
        fill_tab<TR, IO, S, TW>(p, t0 + S, g_base, gpw, lane, reset_first, gb[(h + 1) % kGateDepth], tab[1 - x]);
        if (k + kGateDepth - 1 < n_blocks)
          load_gate_pairs<TR, IO, S>(p, b, t0 + (kGateDepth - 1) * S, g_base, gpw, lane,
                                     gb[(h + kGateDepth - 1) % kGateDepth]);
      }
      __syncthreads();
    }
  }
  if constexpr (SUMMARY) {
    if (streamer && lane_ok) {
#pragma unroll
      for (int v = 0; v < V; ++v)
        *reinterpret_cast<float4*>(p.seg_sum + ((static_cast<int64_t>(b) * p.n_seg + cp.seg) * p.M + m0 + v) * 4) =
            make_float4(Pr[v], CPLX ? Pi[v] : 0.0f, hr[v], CPLX ? hi[v] : 0.0f);
    }
  }
}

// Backward from the saved forward output (no relu epilogue), one chain per
// workgroup in reverse time: lambda_t = dy_t + conj(a_{t+1}) lambda_{t+1},
// dw_t = lambda_t, and dL/da_t = lambda_t conj(h_{t-1}) with h_{t-1} read
// from row t-1 of y (h0 at t = 0).  Wave 0 runs the adjoint and leaves each
// lane's per-step transition gradients in LDS; wave 1 sums them over the
// lanes of each group one block later, applies the polar chain rule (dr,
// dphi) to the group sums and stores the gate gradients.  SUMMARY (time
// segments): the segment's map of the adjoint from zero (P the product of
// conj(a), Q the adjoint leaving its first step) into seg_sum, nothing else;
// otherwise the segment starts from its entering adjoint in seg_state (dlast
// for the last segment, folded in there by the carry kernel).
template <int TR, typename IO, int V, int S, bool SUMMARY = false>
__global__ void __launch_bounds__(128, 1)
chain_bwd_serial_kernel(ScanArgs p) {
  static_assert(!tr_g32(TR), "lane-shared kernels read gates in the I/O dtype");
  if (blockIdx.x == 0 && threadIdx.x == 0) *p.error = 0u;  // no waits here: never an error
  constexpr bool CPLX = TR != TR_REAL;
  constexpr int MB = 64 * V;
  constexpr int R = fast_rounds(S);
  constexpr int TW = (TR == TR_POLAR) ? 4 : (CPLX ? 2 : 1);
  constexpr int ESZ = sizeof(IO);
  constexpr int NG = CPLX ? 2 : 1;    // transition gradients per (step, group)
  constexpr int RED = S * NG + 1;     // padded LDS row of one lane's partials
  using RawT = typename Raw<IO, V>::T;
  __shared__ float tab[2][S * kFastMaxGpw * TW];
  __shared__ float red[2][64 * RED];

  const SerialPos cp = serial_pos(p);
  const int n_blocks = (cp.t_end - cp.t_begin + S - 1) / S;
  if (n_blocks <= 0) return;  // the whole workgroup
  const int lane = threadIdx.x & 63;
  const bool streamer = threadIdx.x < 64;  // wave-uniform
  const int b = cp.b, mb = cp.mb, t_begin = cp.t_begin;
  const int m0 = mb * MB + lane * V;
  const bool lane_ok = m0 < p.M;
  const int gpw = MB / p.gs;
  const int lpg = p.gs / V;
  const int my_g = lane / lpg;
  const int g_base = mb * gpw;
  const bool reset_first = (p.flags & SPARC_FLAG_RESET_FIRST) != 0;
  const uint32_t lane_bytes = static_cast<uint32_t>(lane * V * ESZ);
  const int64_t row0 = static_cast<int64_t>(b) * p.T;
  const int64_t mbase = static_cast<int64_t>(mb) * MB;
  const int64_t stride = static_cast<int64_t>(p.M) * ESZ;

  float xr[V], xi[V];  // conj(a_{t+1}) lambda_{t+1}: the adjoint flowing into step t
  float Pr[V], Pi[V];  // SUMMARY: the product of the segment's conj(a)
  const bool from_seg = !SUMMARY && p.n_seg > 1;
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int64_t i0 = static_cast<int64_t>(b) * p.M + m0 + v;
    const int64_t si = ((static_cast<int64_t>(b) * p.n_seg + cp.seg) * p.M + m0 + v) * 2;
    if (SUMMARY) {
      xr[v] = 0.0f;
      xi[v] = 0.0f;
    } else if (from_seg) {
      xr[v] = (streamer && lane_ok) ? p.seg_state[si] : 0.0f;
      xi[v] = (streamer && CPLX && lane_ok) ? p.seg_state[si + 1] : 0.0f;
    } else {
      xr[v] = (streamer && p.dlast_re && lane_ok) ? p.dlast_re[i0] : 0.0f;
      xi[v] = (streamer && CPLX && p.dlast_im && lane_ok) ? p.dlast_im[i0] : 0.0f;
    }
    Pr[v] = 1.0f;
    Pi[v] = 0.0f;
  }

  // wave 0: dy rows t0 .. t0+S-1 and y rows t0-1 .. t0+S-2 (the state before each step)
  RawT dr[2][S], di[2][S], yr[2][S], yi[2][S];
  GateBlock<S> gb[kGateDepth];  // wave 1: raw gates of iteration j in gb[j % kGateDepth]
  // Unconditional loads, as in the forward: rows are clamped into [0, T-1]
  // and lanes past M read the first element of their mode block; run_block
  // discards what lies outside (dy past T, y before step 0, lanes past M).
  const uint32_t lane_ld = lane_ok ? lane_bytes : 0u;
  auto load_block = [&](int hb, int k) {
    const int t0 = t_begin + k * S;
    const int64_t off = wave_uniform(((row0 + t0) * p.M + mbase) * ESZ);
    const int last = p.T - 1 - t0;  // the block's last step inside T (wave-uniform)
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int sd = s <= last ? s : last;       // dy row t, clamped
      const int sy = max(min(s - 1, last), -t0);  // y row t-1, clamped
      const int64_t od = off + static_cast<int64_t>(sd) * stride;
      const int64_t oy = off + static_cast<int64_t>(sy) * stride;
      dr[hb][s] = ldn<RawT, (SPARC_BWD_NT & 1) != 0>(p.dy_re, od, lane_ld);
      if constexpr (!SUMMARY) yr[hb][s] = ldn<RawT, (SPARC_BWD_NT & 1) != 0>(p.y_re, oy, lane_ld);
      if constexpr (CPLX) {
        di[hb][s] = ldn<RawT, (SPARC_BWD_NT & 1) != 0>(p.dy_im, od, lane_ld);
        if constexpr (!SUMMARY) yi[hb][s] = ldn<RawT, (SPARC_BWD_NT & 1) != 0>(p.y_im, oy, lane_ld);
      }
    }
  };

  // the state before step 0: h0 (fp32) or zero, read once
  float h0r[V], h0i[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int64_t i0 = static_cast<int64_t>(b) * p.M + m0 + v;
    h0r[v] = (streamer && p.h0_re && lane_ok) ? p.h0_re[i0] : 0.0f;
    h0i[v] = (streamer && CPLX && p.h0_im && lane_ok) ? p.h0_im[i0] : 0.0f;
  }
  wait_vm_all();  // the loop-carried adjoint and h0: as in the forward

  auto run_block = [&](int h, int t0, const float* tb, float* rd) {
    const bool edge = t0 == 0 || t0 + S > p.T;  // wave-uniform
    float ar[S], ai[S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
      ar[s] = tb[(s * gpw + my_g) * TW];
      ai[s] = CPLX ? tb[(s * gpw + my_g) * TW + 1] : 0.0f;
    }
    const int64_t off = wave_uniform(((row0 + t0) * p.M + mbase) * ESZ);
#pragma unroll
    for (int s = S - 1; s >= 0; --s) {
      float gy_r[V], gy_i[V], hr[V], hi[V], lr[V], li[V];
      unpack<IO, V>(dr[h][s], gy_r);
      if constexpr (!SUMMARY) unpack<IO, V>(yr[h][s], hr);
      if constexpr (CPLX) {
        unpack<IO, V>(di[h][s], gy_i);
        if constexpr (!SUMMARY) unpack<IO, V>(yi[h][s], hi);
      }
      if (edge) {
        if (t0 + s >= p.T) {  // past T: no incoming gradient (the transition is the identity)
#pragma unroll
          for (int v = 0; v < V; ++v) { gy_r[v] = 0.0f; gy_i[v] = 0.0f; }
        }
        if (t0 + s == 0) {
#pragma unroll
          for (int v = 0; v < V; ++v) { hr[v] = h0r[v]; hi[v] = h0i[v]; }
        }
      }
#pragma unroll
      for (int v = 0; v < V; ++v) {
        lr[v] = gy_r[v] + xr[v];
        if constexpr (CPLX) li[v] = gy_i[v] + xi[v];
      }
      if constexpr (SUMMARY) {  // the adjoint alone; P <- conj(a) P (the identity past T)
#pragma unroll
        for (int v = 0; v < V; ++v) {
          if constexpr (CPLX) {
            xr[v] = fmaf(ar[s], lr[v], ai[s] * li[v]);
            xi[v] = fmaf(ar[s], li[v], -ai[s] * lr[v]);
            const float pr = fmaf(ar[s], Pr[v], ai[s] * Pi[v]);
            Pi[v] = fmaf(ar[s], Pi[v], -ai[s] * Pr[v]);
            Pr[v] = pr;
          } else {
            xr[v] = ar[s] * lr[v];
            Pr[v] *= ar[s];
          }
        }
        continue;
      }
      if (lane_ok && t0 + s < p.T) {
        stn<RawT, (SPARC_BWD_NT & 2) != 0>(p.dw_re, off + s * stride, lane_bytes, pack<IO, V>(lr));
        if constexpr (CPLX) stn<RawT, (SPARC_BWD_NT & 2) != 0>(p.dw_im, off + s * stride, lane_bytes, pack<IO, V>(li));
      }
      float gar = 0.0f, gai = 0.0f;
#pragma unroll
      for (int v = 0; v < V; ++v) {
        if constexpr (CPLX) {
          gar = fmaf(lr[v], hr[v], fmaf(li[v], hi[v], gar));
          gai = fmaf(li[v], hr[v], fmaf(-lr[v], hi[v], gai));
          xr[v] = fmaf(ar[s], lr[v], ai[s] * li[v]);
          xi[v] = fmaf(ar[s], li[v], -ai[s] * lr[v]);
        } else {
          gar = fmaf(lr[v], hr[v], gar);
          xr[v] = ar[s] * lr[v];
        }
      }
      rd[lane * RED + s * NG] = gar;
      if constexpr (CPLX) rd[lane * RED + s * NG + 1] = gai;
    }
  };

  // wave 1: group sums of one block's partials rd (table tb, reset mask rm)
  auto store_block_grads = [&](int t0, const float* tb, const float* rd, uint32_t rm) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int idx = r * 64 + lane;  // pair: step idx / gpw, group idx % gpw
      if (idx < S * gpw) {
        const int step = idx / gpw;
        const int g = idx - step * gpw;
        float sr = 0.0f, si = 0.0f;
        for (int j = 0; j < lpg; ++j) {
          const float* src = rd + (g * lpg + j) * RED + step * NG;
          sr += src[0];
          if constexpr (CPLX) si += src[1];
        }
        const int t = t0 + step;
        if (t < p.T && g_base + g < p.G) {  // the last mode block may hold fewer groups
          float d0 = sr, d1 = si;
          if constexpr (TR == TR_POLAR) {
            const float* e = tb + idx * TW;   // (ar, ai, cos phi, sin phi) of this pair
            d0 = fmaf(sr, e[2], si * e[3]);
            d1 = fmaf(si, e[0], -sr * e[1]);
          }
          // a reset step's transition is the constant 0: no gradient
          const bool reset = (rm >> r) & 1u;
          const int64_t gi = (row0 + t) * p.G + g_base + g;
          store1<IO>(p.dg0, gi, reset ? 0.0f : d0);
          if constexpr (CPLX) store1<IO>(p.dg1, gi, reset ? 0.0f : d1);
        }
      }
    }
  };

  // Iteration j handles block k = n_blocks-1-j with planes, table and
  // partials in buffers x = j & 1.  Wave 1, at iteration j: group sums of
  // block k+1 (table and partials in buffers 1-x), then the table of block
  // k-1 (into buffers 1-x, after those reads), then the gates of block
  // k-(kGateDepth-1).
  uint32_t rm_old = 0u, rm_mid = 0u;  // reset masks: block k+1, block k
  if (streamer) {
    load_block(0, n_blocks - 1);
  } else {
#pragma unroll
    for (int d = 0; d < kGateDepth - 1; ++d)
      if (d < n_blocks)
        load_gate_pairs<TR, IO, S>(p, b, t_begin + (n_blocks - 1 - d) * S, g_base, gpw, lane, gb[d]);
    rm_mid = fill_tab<TR, IO, S, TW>(p, t_begin + (n_blocks - 1) * S, g_base, gpw, lane, reset_first, gb[0], tab[0]);
  }
  __syncthreads();
  for (int j0 = 0; j0 < n_blocks; j0 += kGateDepth) {
#pragma unroll
    for (int h = 0; h < kGateDepth; ++h) {
      const int j = j0 + h;
      if (j >= n_blocks) break;
      const int k = n_blocks - 1 - j;
      const int t0 = t_begin + k * S;
      const int x = h & 1;
      if (streamer) {
        load_block(1 - x, k >= 1 ? k - 1 : 0);  // unconditional, as in the forward
        run_block(x, t0, tab[x], red[x]);
      } else {
        if (!SUMMARY && j >= 1) store_block_grads(t0 + S, tab[1 - x], red[1 - x], rm_old);
        rm_old = rm_mid;
        rm_mid = 0u;
        if (k >= 1) {
          rm_mid = fill_tab<TR, IO, S, TW>(p, t0 - S, g_base, gpw, lane, reset_first,
                                           gb[(h + 1) % kGateDepth], tab[1 - x]);
          if (k >= kGateDepth - 1)
            load_gate_pairs<TR, IO, S>(p, b, t0 - (kGateDepth - 1) * S, g_base, gpw, lane,
                                       gb[(h + kGateDepth - 1) % kGateDepth]);
        }
      }
      __syncthreads();
    }
  }
  if constexpr (SUMMARY) {
    if (streamer && lane_ok) {
#pragma unroll
      for (int v = 0; v < V; ++v)
        *reinterpret_cast<float4*>(p.seg_sum + ((static_cast<int64_t>(b) * p.n_seg + cp.seg) * p.M + m0 + v) * 4) =
            make_float4(Pr[v], CPLX ? Pi[v] : 0.0f, xr[v], CPLX ? xi[v] : 0.0f);
    }
  } else if (streamer) {
    if (lane_ok && p.dh0_re && t_begin == 0) {
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const int64_t i0 = static_cast<int64_t>(b) * p.M + m0 + v;
        p.dh0_re[i0] = xr[v];
        if constexpr (CPLX) p.dh0_im[i0] = xi[v];
      }
    }
  } else {
    const int hl = (n_blocks - 1) & 1;  // buffers of the last iteration (block 0)
    store_block_grads(t_begin, tab[hl], red[hl], rm_old);
  }
}

// ---------------------------------------------------------------------------
// helpers: workspace clear, partial reductions
// ---------------------------------------------------------------------------
#if SPARC_SCAN_OWNS(0)
__global__ void clear_u32_kernel(uint32_t* p, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}
#endif

// out[r, g] = sum_{j < per} part[r, g*per + j] for G columns; fixed order.
template <typename GT>
__global__ void reduce_groups_kernel(const float* part, int64_t rows, int n_mblocks, int G, int per,
                                     void* out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= rows * G) return;
  const int64_t r = i / G;
  const int g = static_cast<int>(i - r * G);
  const float* src = part + r * n_mblocks + static_cast<int64_t>(g) * per;
  float acc = 0.0f;
  for (int j = 0; j < per; ++j) acc += src[j];
  store1<GT>(out, i, acc);
}

}  // namespace sparc

// ===========================================================================
// host side: plans, launchers, C ABI
// ===========================================================================
// This file compiles as one translation unit or, with SPARC_SCAN_PART = k, as
// part k of kScanParts (the build compiles the parts in parallel): part 0
// holds the plan logic and the C ABI, part k >= 1 the launcher of one
// (transition, I/O dtype) pair and every kernel it launches.  Each part sees
// every template; an `extern template` declaration keeps the parts that do
// not own a launcher from instantiating it.
#include <stdio.h>
#include <string.h>

namespace sparc_host {

constexpr int kChunk = 64;  // C = S * NW for every instantiation

// Minimum number of chains for the chain-serial kernels (two resident
// workgroups per CU on a 256-CU MI355X).
constexpr int kChainMin = 512;
constexpr int kSerialMin = 1024;  // one wave per chain: a wave for each of the 1024 SIMDs
// Serial kernels with 4 bf16 modes per lane (8-byte loads per plane): a
// streaming probe of this access pattern on MI355X moved 5.8 TB/s with 512
// such waves against 4.9 TB/s with 1024 waves of 4-byte loads, and fell off
// again at 256 waves.
constexpr int kWideV = 4;
#ifndef SPARC_SERIAL_WIDE_MIN
#define SPARC_SERIAL_WIDE_MIN 512
#endif
constexpr int kSerialWideMin = SPARC_SERIAL_WIDE_MIN;
static_assert(kChunk == sparc::kStateChunk, "one saved-state chunk length");

struct Plan {
  int V = 1;
  int gm = sparc::GATE_LANE;
  bool chain = false;
  bool fast = false;  // chain kernels specialised for lane-shared gates
  bool serial = false;  // one wave per chain (lane-shared gates, many chains)
  bool g32 = false;  // fp32 gates beside bf16 I/O (general kernels only)
  int n_chunks = 0, n_mblocks = 0, n_chains = 0;
  int n_seg = 1, t_seg = 0;  // time segments of the serial kernels (n_seg > 1: few chains)
  int64_t n_tiles = 0;
  size_t flags_off = 0, agg_off = 0, carry_off = 0, part_off = 0, seg_sum_off = 0, seg_state_off = 0, total = 0;
  int64_t part_g_elems = 0, part_p_elems = 0;
};

// steps per prefetched block of the serial kernels (compile-time tunable)
#ifndef SPARC_SERIAL_FWD_S
#define SPARC_SERIAL_FWD_S 16
#endif
#ifndef SPARC_SERIAL_BWD_S
#define SPARC_SERIAL_BWD_S 8
#endif
constexpr int kSerialFwdS = SPARC_SERIAL_FWD_S;
constexpr int kSerialBwdS = SPARC_SERIAL_BWD_S;

// The serial kernels over a plan's chains.  With time segments: the maps of
// every segment but the last one processed (forward 0 .. n-2, backward
// n-1 .. 1), the carry into every segment (from h0 / dlast), then every
// segment from its entering state.
template <int TR, typename IO, int V>
void serial_fwd(const Plan& pl, hipStream_t st, const sparc::ScanArgs& a) {
  const auto ss = reinterpret_cast<sparc_stream_t>(st);
  if (pl.n_seg > 1) {
    const dim3 gs(static_cast<unsigned>(pl.n_chains) * static_cast<unsigned>(pl.n_seg - 1));
    hipLaunchKernelGGL((sparc::chain_fwd_serial_kernel<TR, IO, V, kSerialFwdS, false, true>), gs, dim3(128), 0, st, a);
    // seg_carry refuses B*M > INT32_MAX only; segmented plans have fewer than
    // 512 chains of at most 256 modes, so B*M < 2^17 here
    (void)sparc::seg_carry(a.B, a.M, pl.n_seg, 0, a.seg_sum, a.h0_re, a.h0_im, a.seg_state, ss);
  }
  const dim3 g(static_cast<unsigned>(pl.n_chains) * static_cast<unsigned>(pl.n_seg));
  if ((a.flags & SPARC_FLAG_RELU_OUTPUT) && sparc::tr_kind(TR) != sparc::TR_REAL)
    hipLaunchKernelGGL((sparc::chain_fwd_serial_kernel<TR, IO, V, kSerialFwdS, true>), g, dim3(128), 0, st, a);
  else
    hipLaunchKernelGGL((sparc::chain_fwd_serial_kernel<TR, IO, V, kSerialFwdS, false>), g, dim3(128), 0, st, a);
}
template <int TR, typename IO, int V>
void serial_bwd(const Plan& pl, hipStream_t st, const sparc::ScanArgs& a) {
  const auto ss = reinterpret_cast<sparc_stream_t>(st);
  if (pl.n_seg > 1) {
    sparc::ScanArgs s = a;
    s.seg_lo = 1;
    const dim3 gs(static_cast<unsigned>(pl.n_chains) * static_cast<unsigned>(pl.n_seg - 1));
    hipLaunchKernelGGL((sparc::chain_bwd_serial_kernel<TR, IO, V, kSerialBwdS, true>), gs, dim3(128), 0, st, s);
    (void)sparc::seg_carry(a.B, a.M, pl.n_seg, 1, a.seg_sum, a.dlast_re, a.dlast_im, a.seg_state, ss);  // as above
  }
  const dim3 g(static_cast<unsigned>(pl.n_chains) * static_cast<unsigned>(pl.n_seg));
  hipLaunchKernelGGL((sparc::chain_bwd_serial_kernel<TR, IO, V, kSerialBwdS>), g, dim3(128), 0, st, a);
}

template <int TR, typename IO, int V, int GM>
struct Kernels {
  // look-back kernels: 8 waves x 8 steps
  static constexpr int S = 8;
  static constexpr int NW = kChunk / S;
  // chain-serial kernels
  static constexpr int CS_F = 8, CNW_F = kChunk / CS_F;
  static constexpr int CS_B = 4, CNW_B = kChunk / CS_B;
  static void run(int dir, bool chain, const Plan& pl, hipStream_t st, const sparc::ScanArgs& a) {
    if constexpr (sparc::tr_kind(TR) != sparc::TR_P1 && GM == sparc::GATE_LANE && !sparc::tr_g32(TR)) {
      if (pl.serial && dir == 0) {
        serial_fwd<TR, IO, V>(pl, st, a);
        return;
      }
      if (chain && pl.fast) {
        constexpr int FS = 8, FNW = kChunk / FS;
        const dim3 g(static_cast<unsigned>(pl.n_chains));
        const bool relu = (a.flags & SPARC_FLAG_RELU_OUTPUT) != 0;
        if constexpr (sparc::tr_kind(TR) == sparc::TR_REAL) {
          if (dir == 0) hipLaunchKernelGGL((sparc::chain_fwd_fast_kernel<TR, IO, V, FS, FNW, false>), g, dim3(FNW * 64), 0, st, a);
          else hipLaunchKernelGGL((sparc::chain_bwd_fast_kernel<TR, IO, V, FS, FNW, false>), g, dim3(FNW * 64), 0, st, a);
        } else if (relu) {
          if (dir == 0) hipLaunchKernelGGL((sparc::chain_fwd_fast_kernel<TR, IO, V, FS, FNW, true>), g, dim3(FNW * 64), 0, st, a);
          else hipLaunchKernelGGL((sparc::chain_bwd_fast_kernel<TR, IO, V, FS, FNW, true>), g, dim3(FNW * 64), 0, st, a);
        } else {
          if (dir == 0) hipLaunchKernelGGL((sparc::chain_fwd_fast_kernel<TR, IO, V, FS, FNW, false>), g, dim3(FNW * 64), 0, st, a);
          else hipLaunchKernelGGL((sparc::chain_bwd_fast_kernel<TR, IO, V, FS, FNW, false>), g, dim3(FNW * 64), 0, st, a);
        }
        return;
      }
    }
    return run_general(dir, chain, pl, st, a);
  }
  // backward from the saved forward output (no relu epilogue); false when
  // this plan has no such kernel and the caller must fall back to w
  static bool run_saved(const Plan& pl, hipStream_t st, const sparc::ScanArgs& a) {
    if (!pl.chain) {  // look-back tiles, any transition and gate layout
      const dim3 g(static_cast<unsigned>(pl.n_tiles));
      hipLaunchKernelGGL((sparc::scan_bwd_kernel<TR, IO, V, GM, S, NW, true>), g, dim3(NW * 64), 0, st, a);
      return true;
    }
    if constexpr (sparc::tr_kind(TR) != sparc::TR_P1 && GM == sparc::GATE_LANE && !sparc::tr_g32(TR)) {
      if (pl.serial) {
        serial_bwd<TR, IO, V>(pl, st, a);
        return true;
      }
      if (pl.chain && pl.fast) {
        constexpr int FS = 8, FNW = kChunk / FS;
        const dim3 g(static_cast<unsigned>(pl.n_chains));
        hipLaunchKernelGGL((sparc::chain_bwd_saved_kernel<TR, IO, V, FS, FNW>), g, dim3(FNW * 64), 0, st, a);
        return true;
      }
    }
    return false;
  }
  static void run_general(int dir, bool chain, const Plan& pl, hipStream_t st, const sparc::ScanArgs& a) {
    if (chain) {
      const dim3 g(static_cast<unsigned>(pl.n_chains));
      if (dir == 0)
        hipLaunchKernelGGL((sparc::chain_fwd_kernel<TR, IO, V, GM, CS_F, CNW_F>), g, dim3(CNW_F * 64), 0, st, a);
      else
        hipLaunchKernelGGL((sparc::chain_bwd_kernel<TR, IO, V, GM, CS_B, CNW_B>), g, dim3(CNW_B * 64), 0, st, a);
      return;
    }
    const dim3 g(static_cast<unsigned>(pl.n_tiles));
    if (dir == 0) hipLaunchKernelGGL((sparc::scan_fwd_kernel<TR, IO, V, GM, S, NW>), g, dim3(NW * 64), 0, st, a);
    else hipLaunchKernelGGL((sparc::scan_bwd_kernel<TR, IO, V, GM, S, NW, false>), g, dim3(NW * 64), 0, st, a);
  }
};

// dir 0: forward, 1: backward (recomputing states from w), 2: backward from
// the saved forward output if this plan has a kernel for it (returns false
// without launching anything otherwise)
template <int TR, typename IO>
bool launch_v(int dir, const Plan& pl, hipStream_t st, const sparc::ScanArgs& a) {
  constexpr int VM = (sparc::tr_kind(TR) == sparc::TR_REAL) ? 4 : 2;
  const int V = pl.V, gm = pl.gm;
#define SPARC_LAUNCH(VV, GG)                                                            \
  if (V == VV && gm == GG) {                                                           \
    if (dir == 2) return Kernels<TR, IO, VV, GG>::run_saved(pl, st, a);                  \
    Kernels<TR, IO, VV, GG>::run(dir, pl.chain, pl, st, a);                              \
    return true;                                                                        \
  }
  if constexpr ((sparc::tr_kind(TR) == sparc::TR_POLAR || sparc::tr_kind(TR) == sparc::TR_CART) &&
                sparc::IsBf16<IO>::value && !sparc::tr_g32(TR)) {
    if (V == kWideV) {
      if (!pl.serial || gm != sparc::GATE_LANE) return false;
      if (dir == 1) return false;  // no recomputing kernel: wide plans need the saved output
      if (dir == 2) serial_bwd<TR, IO, kWideV>(pl, st, a);
      else serial_fwd<TR, IO, kWideV>(pl, st, a);
      return true;
    }
  }
  SPARC_LAUNCH(VM, sparc::GATE_LANE)
  SPARC_LAUNCH(VM, sparc::GATE_CROSS)
  SPARC_LAUNCH(1, sparc::GATE_LANE)
  SPARC_LAUNCH(1, sparc::GATE_CROSS)
  if constexpr (sparc::tr_kind(TR) == sparc::TR_CART || sparc::tr_kind(TR) == sparc::TR_REAL) {
    SPARC_LAUNCH(VM, sparc::GATE_MODE)
    SPARC_LAUNCH(1, sparc::GATE_MODE)
  }
#undef SPARC_LAUNCH
  return false;
}

// Launchers by part.  TR | TR_G32: fp32 gates beside bf16 I/O.
#define SPARC_LV(TRV, IOT) bool launch_v<TRV, IOT>(int, const Plan&, hipStream_t, const sparc::ScanArgs&)
#if SPARC_SCAN_OWNS(1)
template SPARC_LV(sparc::TR_P1, float);
#else
extern template SPARC_LV(sparc::TR_P1, float);
#endif
#if SPARC_SCAN_OWNS(2)
template SPARC_LV(sparc::TR_P1, sparc::bf16);
#else
extern template SPARC_LV(sparc::TR_P1, sparc::bf16);
#endif
#if SPARC_SCAN_OWNS(3)
template SPARC_LV(sparc::TR_POLAR, float);
#else
extern template SPARC_LV(sparc::TR_POLAR, float);
#endif
#if SPARC_SCAN_OWNS(4)
template SPARC_LV(sparc::TR_POLAR, sparc::bf16);
#else
extern template SPARC_LV(sparc::TR_POLAR, sparc::bf16);
#endif
#if SPARC_SCAN_OWNS(5)
template SPARC_LV(sparc::TR_CART, float);
#else
extern template SPARC_LV(sparc::TR_CART, float);
#endif
#if SPARC_SCAN_OWNS(6)
template SPARC_LV(sparc::TR_CART, sparc::bf16);
#else
extern template SPARC_LV(sparc::TR_CART, sparc::bf16);
#endif
#if SPARC_SCAN_OWNS(7)
template SPARC_LV(sparc::TR_REAL, float);
#else
extern template SPARC_LV(sparc::TR_REAL, float);
#endif
#if SPARC_SCAN_OWNS(8)
template SPARC_LV(sparc::TR_REAL, sparc::bf16);
#else
extern template SPARC_LV(sparc::TR_REAL, sparc::bf16);
#endif
#if SPARC_SCAN_OWNS(9)
template SPARC_LV(sparc::TR_POLAR | sparc::TR_G32, sparc::bf16);
#else
extern template SPARC_LV(sparc::TR_POLAR | sparc::TR_G32, sparc::bf16);
#endif
#if SPARC_SCAN_OWNS(10)
template SPARC_LV(sparc::TR_CART | sparc::TR_G32, sparc::bf16);
#else
extern template SPARC_LV(sparc::TR_CART | sparc::TR_G32, sparc::bf16);
#endif
#if SPARC_SCAN_OWNS(11)
template SPARC_LV(sparc::TR_REAL | sparc::TR_G32, sparc::bf16);
#else
extern template SPARC_LV(sparc::TR_REAL | sparc::TR_G32, sparc::bf16);
#endif
#undef SPARC_LV

}  // namespace sparc_host

#if SPARC_SCAN_OWNS(0)
namespace {

using namespace sparc_host;

sparc_status fail(sparc_status s, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
sparc_status fail(sparc_status s, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(sparc::error_buffer(), 512, fmt, ap);
  va_end(ap);
  return s;
}

// Polls each cross-workgroup wait of the look-back kernels makes before it
// gives up (sets the workspace error word and lets the workgroup finish).
static std::atomic<uint32_t> g_wait_limit{1u << 20};
}  // namespace

namespace sparc {
uint32_t wait_limit() { return g_wait_limit.load(std::memory_order_relaxed); }
}  // namespace sparc

namespace {

bool is_pow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }

// Time segments of the serial kernels: below kSegChains chains (where the
// look-back kernels would run), T splits into segments of a multiple of 64
// steps, at least kSegMinSteps long, enough for about kSegTarget workgroups
// (per direction: at B=1, T=65536, M=2048 the forward took 0.376 / 0.397 /
// 0.426 ms with 512 / 1024 / 2048 workgroups, the backward 0.524 / 0.479 /
// 0.489 ms).
#ifndef SPARC_SERIAL_SEG_CHAINS
#define SPARC_SERIAL_SEG_CHAINS 512
#endif
#ifndef SPARC_SERIAL_SEG_TARGET_FWD
#define SPARC_SERIAL_SEG_TARGET_FWD 512
#endif
#ifndef SPARC_SERIAL_SEG_TARGET_BWD
#define SPARC_SERIAL_SEG_TARGET_BWD 1024
#endif
#ifndef SPARC_SERIAL_SEG_MIN
#define SPARC_SERIAL_SEG_MIN 256
#endif
constexpr int64_t kSegChains = SPARC_SERIAL_SEG_CHAINS;
constexpr int64_t kSegTarget[2] = {SPARC_SERIAL_SEG_TARGET_FWD, SPARC_SERIAL_SEG_TARGET_BWD};
constexpr int64_t kSegMinSteps = SPARC_SERIAL_SEG_MIN;
static_assert(kSegMinSteps % 64 == 0 && kSegChains <= kSegTarget[0] && kSegChains <= kSegTarget[1],
              "segments of whole chunks, at least two");

bool want_segments(int64_t chains, int64_t T, int64_t below = kSegChains) {
  return chains < below && T >= 2 * kSegMinSteps;
}

// n >= 2 segments of t_seg steps (a multiple of the saved-state chunk), or 1
void choose_serial_segments(int direction, int64_t below, int64_t chains, int64_t T, int& n_seg, int& t_seg) {
  n_seg = 1;
  t_seg = static_cast<int>(T);
  if (!want_segments(chains, T, below)) return;
  const int64_t target = kSegTarget[direction ? 1 : 0];
  int64_t n = std::min((target + chains - 1) / chains, T / kSegMinSteps);
  if (n < 2) return;
  int64_t len = (T + n - 1) / n;
  len = (len + kChunk - 1) / kChunk * kChunk;
  n = (T + len - 1) / len;
  if (n < 2) return;
  n_seg = static_cast<int>(n);
  t_seg = static_cast<int>(len);
}

// Chain-count thresholds of the automatic plan for lane-shared gates (chains
// at the plan's modes per lane).  Measured fwd+bwd, polar and real, G = M/16,
// B*T*M = 2^28, chains 8 .. 1024:
//   bf16 complex: wide (4 modes) serial from 512 wide chains (69-72 % of 8
//     TB/s), the 8-wave chain kernels at 2 modes from 128 wide chains (53-54 %
//     against 46-48 % segmented), segments below (43-48 %; look-back 29-33 %);
//   bf16 real (4 modes): serial from 1024 chains (75 %), chain kernels from
//     256 (59-61 %; segments 41 %), segments below (41-44 %; look-back 31-39 %);
//   fp32 complex (2 modes): serial from 512 chains (63-65 %), look-back below
//     (53-62 %; segments 46-52 %, chain kernels 29-54 %);
//   fp32 real (4 modes): look-back everywhere (60-77 %; serial 53-75 %).
// A backward without the saved output (recompute) has no serial kernel of its
// own: fp32 then keeps the look-back.
constexpr int64_t kSegBelowCplx = 128;  // bf16 complex: segments below this many wide chains
constexpr int64_t kSegBelowReal = 256;  // bf16 real
constexpr int64_t kNever = INT64_MAX;
void plan_lane_shared(bool cplx, bool bf16, bool wide, bool recompute_bwd, int64_t& seg_below, int64_t& serial_min,
                      int64_t& chain_min) {
  if (bf16) {
    seg_below = cplx ? kSegBelowCplx : kSegBelowReal;
    serial_min = cplx && wide ? kSerialWideMin : kSerialMin;
    chain_min = 256;
  } else {
    seg_below = 0;
    serial_min = cplx && !recompute_bwd ? 512 : kNever;
    chain_min = kNever;
  }
}

// Chooses V and the gate mode; fills sizes.  Returns an error message or NULL.
// allow_wide: the caller can use the 4-mode serial kernels (their pointers are
// 8-byte aligned and, backward, the states come from the saved output).
// allow_seg: the serial kernels may split time into segments (backward: the
// states come from the saved output).
const char* make_plan(const sparc_scan_desc* d, int direction, Plan* pl, bool allow_wide = true,
                      bool allow_seg = true) {
  if (!d) return "desc is NULL";
  if (d->batch <= 0 || d->length < 0 || d->modes <= 0 || d->groups <= 0) return "B, M, G must be > 0 and T >= 0";
  if (d->modes % d->groups) return "groups must divide modes";
  if (d->transition < 0 || d->transition > 3) return "unknown transition";
  if (d->io_dtype != SPARC_F32 && d->io_dtype != SPARC_BF16) return "unknown io_dtype";
  const bool p1 = d->transition == SPARC_TRANSITION_P1;
  if (d->gate_dtype != SPARC_F32 && d->gate_dtype != SPARC_BF16) return "unknown gate_dtype";
  if (p1 && d->gate_dtype != SPARC_F32) return "P1 gates (eta, delta) must be fp32";
  // fp32 gates beside bf16 I/O: the general (per-lane transition) kernels
  const bool g32 = !p1 && d->gate_dtype == SPARC_F32 && d->io_dtype == SPARC_BF16;
  if (!p1 && d->gate_dtype != d->io_dtype && !g32) return "bf16 gates need bf16 I/O";
  if ((d->flags & SPARC_FLAG_RELU_OUTPUT) && d->transition == SPARC_TRANSITION_REAL)
    return "RELU_OUTPUT needs a complex transition";
  if (d->batch * d->length * d->modes * 2 >= (int64_t(1) << 62)) return "tensor too large";
  if (d->modes > INT32_MAX / 2 || d->length > INT32_MAX - kChunk || d->batch > INT32_MAX) return "dimension too large";
  const int64_t M = d->modes, G = d->groups, gs = M / G;
  const int vmax = (d->transition == SPARC_TRANSITION_REAL) ? 4 : 2;
  int V = 0, gm = 0;
  auto try_v = [&](int v) -> bool {
    if (M % v) return false;
    if (gs == 1 && (d->transition == SPARC_TRANSITION_CARTESIAN || d->transition == SPARC_TRANSITION_REAL)) {
      V = v; gm = sparc::GATE_MODE; return true;
    }
    if (gs % v) return false;
    const int64_t mbm = 64 * v;
    if (G == 1 || gs % mbm == 0) { V = v; gm = sparc::GATE_CROSS; return true; }
    if (mbm % gs == 0 && is_pow2(gs / v)) { V = v; gm = sparc::GATE_LANE; return true; }
    return false;
  };
  const bool force_l = (d->flags & SPARC_FLAG_ALGO_LOOKBACK) != 0;
  const bool force_c = (d->flags & SPARC_FLAG_ALGO_CHAIN) != 0;
  const bool force_s = (d->flags & SPARC_FLAG_ALGO_SERIAL) != 0;
  if (int(force_l) + int(force_c) + int(force_s) > 1)
    return "ALGO_LOOKBACK, ALGO_CHAIN and ALGO_SERIAL are exclusive";
  const bool auto_plan = !force_l && !force_c && !force_s;
  const bool cplx_tr = d->transition != SPARC_TRANSITION_REAL;
  const bool bf16_io = d->io_dtype == SPARC_BF16;
  // Complex bf16 with lane-shared gates: the serial kernels stream 8 bytes
  // per lane and plane (4 modes) when that still leaves enough chains, or
  // over time segments when the chains are few.
  bool wide = false;
  if (!p1 && !g32 && cplx_tr && bf16_io && M % kWideV == 0 &&
      gs % kWideV == 0 && (64 * kWideV) % gs == 0 && is_pow2(gs / kWideV) &&
      (64 * kWideV) / gs <= sparc::kFastMaxGpw && !force_l && !force_c && allow_wide) {
    const int64_t chains = d->batch * ((M + 64 * kWideV - 1) / (64 * kWideV));
    wide = force_s || chains >= kSerialWideMin || (allow_seg && want_segments(chains, d->length, kSegBelowCplx));
  }
  if (wide) {
    V = kWideV;
    gm = sparc::GATE_LANE;
  } else if (!try_v(vmax) && !try_v(1)) {
    return "unsupported gate group size (need G == 1, M/G == 1, M/G dividing 64*V or a multiple of it)";
  }
  pl->V = V;
  pl->gm = gm;
  pl->g32 = g32;
  pl->n_chunks = static_cast<int>((d->length + kChunk - 1) / kChunk);
  pl->n_mblocks = static_cast<int>((M + 64 * V - 1) / (64 * V));
  pl->n_chains = static_cast<int>(d->batch * pl->n_mblocks);
  pl->n_tiles = static_cast<int64_t>(pl->n_chains) * pl->n_chunks;
  const bool lane_shared = !p1 && !g32 && gm == sparc::GATE_LANE && (64 * V) / gs <= sparc::kFastMaxGpw;
  // The automatic plan for lane-shared gates, by I/O dtype and transition
  // (MI355X, fwd+bwd at B*T*M = 2^28, G = M/16; `plan_lane_shared` below):
  // bf16 streams half the bytes per tile, so the look-back's per-tile cost
  // weighs twice and the chain, serial and segmented serial kernels win;
  // fp32 tiles carry enough bytes for the look-back to win below the serial
  // kernels' chain count, and for real scans everywhere.
  int64_t seg_below = 0, serial_min = kSerialMin, chain_min = kChainMin;
  if (force_s) {
    seg_below = kSegChains;
  } else if (auto_plan && lane_shared) {
    plan_lane_shared(cplx_tr, bf16_io, wide, direction == 1 && !allow_seg, seg_below, serial_min, chain_min);
  }
  pl->n_seg = 1;
  pl->t_seg = static_cast<int>(d->length);
  if (allow_seg && lane_shared && seg_below > 0 && (wide || !cplx_tr || force_s))
    choose_serial_segments(direction, seg_below, pl->n_chains, d->length, pl->n_seg, pl->t_seg);
  pl->serial = wide || pl->n_seg > 1 || (lane_shared && (force_s || (auto_plan && pl->n_chains >= serial_min)));
  pl->chain = pl->serial || force_c || force_s || (auto_plan && pl->n_chains >= chain_min);
  pl->fast = pl->chain && lane_shared;
  const bool cplx = d->transition != SPARC_TRANSITION_REAL;
  const int NQ = cplx ? 4 : 2, NH = cplx ? 2 : 1;
  // [0] ticket, [1] error; then, for look-back only, one flag and one
  // aggregate per tile and (backward) the carries; then gradient partials.
  size_t off = 256;
  pl->flags_off = off;
  if (!pl->chain) off += ((static_cast<size_t>(pl->n_tiles) * 4 + 255) / 256) * 256;
  pl->agg_off = off;
  if (!pl->chain) off += ((static_cast<size_t>(pl->n_tiles) * 64 * V * NQ * 4 + 255) / 256) * 256;
  pl->carry_off = off;
  if (direction == 1 && !pl->chain)
    off += ((static_cast<size_t>(d->batch) * pl->n_chunks * M * NH * 4 + 255) / 256) * 256;
  pl->part_off = off;
  pl->part_g_elems = 0;
  pl->part_p_elems = 0;
  if (direction == 1) {
    if (gm == sparc::GATE_CROSS) pl->part_g_elems = d->batch * d->length * pl->n_mblocks;
    // P1 nu/theta partials: one row per tile (look-back) or per batch row (chain)
    if (p1) pl->part_p_elems = d->batch * static_cast<int64_t>(pl->chain ? 1 : pl->n_chunks) * M;
    off += ((static_cast<size_t>(2 * pl->part_g_elems + 2 * pl->part_p_elems) * 4 + 255) / 256) * 256;
  }
  if (pl->n_seg > 1) {  // each segment's map [B][n_seg][M][4], its entering state [B][n_seg][M][2]
    pl->seg_sum_off = off;
    off += ((static_cast<size_t>(d->batch) * pl->n_seg * M * 16 + 255) / 256) * 256;
    pl->seg_state_off = off;
    off += ((static_cast<size_t>(d->batch) * pl->n_seg * M * 8 + 255) / 256) * 256;
  }
  pl->total = off;
  return nullptr;
}

bool launch(int dir, const sparc_scan_desc* d, const Plan& pl, hipStream_t st, const sparc::ScanArgs& a) {
  const bool bf = d->io_dtype == SPARC_BF16;
  switch (d->transition) {
    case SPARC_TRANSITION_P1:
      return bf ? launch_v<sparc::TR_P1, sparc::bf16>(dir, pl, st, a)
                : launch_v<sparc::TR_P1, float>(dir, pl, st, a);
    case SPARC_TRANSITION_POLAR:
      if (pl.g32) return launch_v<sparc::TR_POLAR | sparc::TR_G32, sparc::bf16>(dir, pl, st, a);
      return bf ? launch_v<sparc::TR_POLAR, sparc::bf16>(dir, pl, st, a)
                : launch_v<sparc::TR_POLAR, float>(dir, pl, st, a);
    case SPARC_TRANSITION_CARTESIAN:
      if (pl.g32) return launch_v<sparc::TR_CART | sparc::TR_G32, sparc::bf16>(dir, pl, st, a);
      return bf ? launch_v<sparc::TR_CART, sparc::bf16>(dir, pl, st, a)
                : launch_v<sparc::TR_CART, float>(dir, pl, st, a);
    default:
      if (pl.g32) return launch_v<sparc::TR_REAL | sparc::TR_G32, sparc::bf16>(dir, pl, st, a);
      return bf ? launch_v<sparc::TR_REAL, sparc::bf16>(dir, pl, st, a)
                : launch_v<sparc::TR_REAL, float>(dir, pl, st, a);
  }
}

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }
bool aligned8(const void* p) { return aligned(p, 8); }  // NULL counts as aligned

}  // namespace

extern "C" {

const char* sparc_last_error(void) { return sparc::error_buffer(); }
const char* sparc_version(void) { return "sparc_hip 0.1 gfx950"; }

int64_t sparc_scan_chunk_length(const sparc_scan_desc*) { return kChunk; }

int64_t sparc_scan_chunk_count(const sparc_scan_desc* d) {
  if (!d || d->length < 0) return -1;
  return (d->length + kChunk - 1) / kChunk;
}

size_t sparc_scan_workspace_bytes(const sparc_scan_desc* d, int direction) {
  // enough for every plan: the call decides from its pointers
  size_t n = 0;
  for (int k = 0; k < 4; ++k) {
    Plan pk;
    if (make_plan(d, direction, &pk, (k & 1) != 0, (k & 2) != 0)) return 0;
    n = pk.total > n ? pk.total : n;
  }
  const size_t f = sparc::p1_fused_workspace_bytes(d, direction);
  return f > n ? f : n;
}

// The P1 scan with one gate pair per token takes the one-wave-per-chain
// kernels of the fused module path (p1_fused.h) when nothing needs the
// general kernels: aligned planes, a large enough workspace.  Otherwise the
// general kernels run.
static bool p1_fused_route(const sparc_scan_desc* d, int direction, const void* const* planes, int n_planes,
                           const float* chunk_state, size_t workspace_bytes) {
  if (!sparc::p1_fused_shape(d)) return false;
  if (workspace_bytes < sparc::p1_fused_workspace_bytes(d, direction)) return false;
  for (int i = 0; i < n_planes; ++i)
    if (!aligned(planes[i], 8)) return false;
  return aligned(chunk_state, 16);
}

static sparc_status common_checks(const sparc_scan_desc* d, int dir, Plan* pl,
                                  void* workspace, size_t workspace_bytes, bool allow_wide, bool allow_seg) {
  if (const char* e = make_plan(d, dir, pl, allow_wide, allow_seg)) return fail(SPARC_EINVAL, "%s", e);
  if (!workspace) return fail(SPARC_EWORKSPACE, "workspace is NULL");
  if (workspace_bytes < pl->total)
    return fail(SPARC_EWORKSPACE, "workspace too small: %zu < %zu", workspace_bytes, pl->total);
  if (!aligned(workspace, 256)) return fail(SPARC_EINVAL, "workspace must be 256-byte aligned");
  return SPARC_OK;
}

static void fill_ws(sparc::ScanArgs& a, const Plan& pl, void* ws) {
  char* base = static_cast<char*>(ws);
  a.ticket = reinterpret_cast<uint32_t*>(base);
  a.error = reinterpret_cast<uint32_t*>(base) + 1;
  a.flagv = reinterpret_cast<uint32_t*>(base + pl.flags_off);
  a.agg = reinterpret_cast<float*>(base + pl.agg_off);
  a.carry = reinterpret_cast<float*>(base + pl.carry_off);
  float* part = reinterpret_cast<float*>(base + pl.part_off);
  a.part_g0 = part;
  a.part_g1 = part + pl.part_g_elems;
  a.part_nu = part + 2 * pl.part_g_elems;
  a.part_theta = part + 2 * pl.part_g_elems + pl.part_p_elems;
  a.n_seg = pl.n_seg;
  a.t_seg = pl.t_seg;
  a.seg_lo = 0;
  a.seg_sum = pl.n_seg > 1 ? reinterpret_cast<float*>(base + pl.seg_sum_off) : nullptr;
  a.seg_state = pl.n_seg > 1 ? reinterpret_cast<float*>(base + pl.seg_state_off) : nullptr;
}

static sparc_status clear_ws(const Plan& pl, void* ws, hipStream_t st) {
  // ticket + error words and one flag per tile
  char* base = static_cast<char*>(ws);
  hipLaunchKernelGGL(sparc::clear_u32_kernel, dim3(1), dim3(64), 0, st,
                     reinterpret_cast<uint32_t*>(base), int64_t(64));
  const int64_t n = pl.n_tiles;
  if (n > 0)
    hipLaunchKernelGGL(sparc::clear_u32_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, st,
                       reinterpret_cast<uint32_t*>(base + pl.flags_off), n);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(SPARC_EHIP, "clear launch: %s", hipGetErrorString(e));
  return SPARC_OK;
}

static sparc_status check_ptrs(size_t esz, const Plan& pl, const void* const* ptrs, int n) {
  for (int i = 0; i < n; ++i)
    if (ptrs[i] && !aligned(ptrs[i], esz * pl.V))
      return fail(SPARC_EINVAL, "tensor %d not aligned to %zu bytes", i, esz * pl.V);
  return SPARC_OK;
}

static sparc_status check_io_ptrs(const sparc_scan_desc* d, const Plan& pl, const void* const* ptrs, int n) {
  return check_ptrs(d->io_dtype == SPARC_BF16 ? 2 : 4, pl, ptrs, n);
}

static sparc_status check_gate_ptrs(const sparc_scan_desc* d, const Plan& pl, const void* const* ptrs, int n) {
  return check_ptrs(d->gate_dtype == SPARC_BF16 ? 2 : 4, pl, ptrs, n);
}

sparc_status sparc_scan_forward(const sparc_scan_desc* d, const void* gate0, const void* gate1,
                                const float* nu_log, const float* theta_log,
                                const void* w_re, const void* w_im,
                                const float* h0_re, const float* h0_im,
                                const int32_t* segment_pos,
                                void* y_re, void* y_im, float* chunk_state,
                                void* workspace, size_t workspace_bytes, sparc_stream_t stream) {
  Plan pl;
  const bool wide_ok = aligned8(w_re) && aligned8(w_im) && aligned8(y_re) && aligned8(y_im);
  if (sparc_status s = common_checks(d, 0, &pl, workspace, workspace_bytes, wide_ok, true)) return s;
  if (d->length == 0) return SPARC_OK;  // nothing to read or write
  const bool cplx = d->transition != SPARC_TRANSITION_REAL;
  const bool relu = (d->flags & SPARC_FLAG_RELU_OUTPUT) != 0;
  if (!gate0 || !w_re || !y_re || !chunk_state) return fail(SPARC_EINVAL, "gate0, w_re, y_re, chunk_state are required");
  if (cplx && (!gate1 || !w_im)) return fail(SPARC_EINVAL, "complex transitions need gate1 and w_im");
  if (cplx && !relu && !y_im) return fail(SPARC_EINVAL, "y_im is required");
  if (d->transition == SPARC_TRANSITION_P1 && (!nu_log || !theta_log)) return fail(SPARC_EINVAL, "P1 needs nu_log, theta_log");
  if (cplx && ((h0_re == nullptr) != (h0_im == nullptr))) return fail(SPARC_EINVAL, "h0_re/h0_im must both be given");
  const void* ptrs[] = {w_re, w_im, y_re, relu ? nullptr : y_im};
  if (sparc_status s = check_io_ptrs(d, pl, ptrs, 4)) return s;
  if (pl.gm == sparc::GATE_MODE) {
    const void* gp[] = {gate0, gate1};
    if (sparc_status s = check_gate_ptrs(d, pl, gp, 2)) return s;
  }
  if (!aligned(chunk_state, 8 * pl.V)) return fail(SPARC_EINVAL, "chunk_state must be %d-byte aligned", 8 * pl.V);
  {
    const void* fp[] = {w_re, w_im, y_re, y_im, h0_re, h0_im};
    if (p1_fused_route(d, 0, fp, 6, chunk_state, workspace_bytes))
      return sparc::p1_fused_forward(d, static_cast<const float*>(gate0), static_cast<const float*>(gate1), nu_log,
                                     theta_log, w_re, w_im, h0_re, h0_im, segment_pos, y_re, relu ? nullptr : y_im,
                                     chunk_state, workspace, workspace_bytes, stream);
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (!pl.chain)
    if (sparc_status s = clear_ws(pl, workspace, st)) return s;
  sparc::ScanArgs a{};
  a.B = static_cast<int>(d->batch);
  a.T = static_cast<int>(d->length);
  a.M = static_cast<int>(d->modes);
  a.G = static_cast<int>(d->groups);
  a.gs = static_cast<int>(d->modes / d->groups);
  a.n_chunks = pl.n_chunks;
  a.n_mblocks = pl.n_mblocks;
  a.n_chains = pl.n_chains;
  a.flags = static_cast<uint32_t>(d->flags);
  a.spin_limit = g_wait_limit.load(std::memory_order_relaxed);
  a.g0 = gate0; a.g1 = gate1; a.nu_log = nu_log; a.theta_log = theta_log;
  a.w_re = w_re; a.w_im = w_im; a.h0_re = h0_re; a.h0_im = h0_im; a.segpos = segment_pos;
  a.y_re = y_re; a.y_im = y_im; a.chunk_state = chunk_state;
  fill_ws(a, pl, workspace);
  if (!launch(0, d, pl, st, a)) return fail(SPARC_EUNSUPPORTED, "no forward kernel for this plan");
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(SPARC_EHIP, "scan forward launch: %s", hipGetErrorString(e));
  return SPARC_OK;
}

// T == 0: no step touches the state, so dh0 = dlast and the parameter
// gradients are zero.
static sparc_status empty_backward(const sparc_scan_desc* d, const float* dlast_re, const float* dlast_im,
                                   float* dnu_log, float* dtheta_log, float* dh0_re, float* dh0_im,
                                   hipStream_t st) {
  const int64_t bm = d->batch * d->modes;
  const dim3 gb(static_cast<unsigned>((bm + 255) / 256)), gm(static_cast<unsigned>((d->modes + 255) / 256));
  hipError_t ce = hipSuccess;
  if (dh0_re) {
    if (dlast_re) ce = hipMemcpyAsync(dh0_re, dlast_re, bm * 4, hipMemcpyDeviceToDevice, st);
    else hipLaunchKernelGGL(sparc::clear_u32_kernel, gb, dim3(256), 0, st, reinterpret_cast<uint32_t*>(dh0_re), bm);
  }
  if (dh0_im && ce == hipSuccess) {
    if (dlast_im) ce = hipMemcpyAsync(dh0_im, dlast_im, bm * 4, hipMemcpyDeviceToDevice, st);
    else hipLaunchKernelGGL(sparc::clear_u32_kernel, gb, dim3(256), 0, st, reinterpret_cast<uint32_t*>(dh0_im), bm);
  }
  if (ce != hipSuccess) return fail(SPARC_EHIP, "empty backward copy: %s", hipGetErrorString(ce));
  if (dnu_log) hipLaunchKernelGGL(sparc::clear_u32_kernel, gm, dim3(256), 0, st, reinterpret_cast<uint32_t*>(dnu_log), d->modes);
  if (dtheta_log) hipLaunchKernelGGL(sparc::clear_u32_kernel, gm, dim3(256), 0, st, reinterpret_cast<uint32_t*>(dtheta_log), d->modes);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? SPARC_OK : fail(SPARC_EHIP, "empty backward: %s", hipGetErrorString(e));
}

sparc_status sparc_scan_backward(const sparc_scan_desc* d, const void* gate0, const void* gate1,
                                 const float* nu_log, const float* theta_log,
                                 const void* w_re, const void* w_im,
                                 const void* y_re, const void* y_im,
                                 const float* h0_re, const float* h0_im,
                                 const int32_t* segment_pos, const float* chunk_state,
                                 const void* dy_re, const void* dy_im,
                                 const float* dlast_re, const float* dlast_im,
                                 void* dw_re, void* dw_im, void* dgate0, void* dgate1,
                                 float* dnu_log, float* dtheta_log,
                                 float* dh0_re, float* dh0_im,
                                 void* workspace, size_t workspace_bytes, sparc_stream_t stream) {
  Plan pl;
  const bool relu = d && (d->flags & SPARC_FLAG_RELU_OUTPUT) != 0;
  // the 4-mode serial backward reads the states from the saved output
  const bool wide_ok = y_re && !relu && aligned8(w_re) && aligned8(w_im) && aligned8(y_re) &&
                       aligned8(y_im) && aligned8(dy_re) && aligned8(dy_im) && aligned8(dw_re) &&
                       aligned8(dw_im);
  if (sparc_status s = common_checks(d, 1, &pl, workspace, workspace_bytes, wide_ok, y_re && !relu)) return s;
  const bool cplx = d->transition != SPARC_TRANSITION_REAL;
  const bool p1 = d->transition == SPARC_TRANSITION_P1;
  if (d->length == 0) {
    if (p1 && (!dnu_log || !dtheta_log)) return fail(SPARC_EINVAL, "P1 needs dnu_log, dtheta_log");
    if (cplx && ((dh0_re == nullptr) != (dh0_im == nullptr))) return fail(SPARC_EINVAL, "dh0_re/dh0_im must both be given");
    return empty_backward(d, dlast_re, dlast_im, dnu_log, dtheta_log, dh0_re, dh0_im,
                          reinterpret_cast<hipStream_t>(stream));
  }
  if (!gate0 || !w_re || !dy_re || !dw_re || !dgate0 || !chunk_state)
    return fail(SPARC_EINVAL, "gate0, w_re, dy_re, dw_re, dgate0, chunk_state are required");
  if (cplx && (!gate1 || !w_im || !dw_im || !dgate1)) return fail(SPARC_EINVAL, "complex transitions need gate1, w_im, dw_im, dgate1");
  if (cplx && !relu && !dy_im) return fail(SPARC_EINVAL, "dy_im is required");
  if (p1 && (!nu_log || !theta_log || !dnu_log || !dtheta_log)) return fail(SPARC_EINVAL, "P1 needs nu_log, theta_log, dnu_log, dtheta_log");
  if (cplx && ((dh0_re == nullptr) != (dh0_im == nullptr))) return fail(SPARC_EINVAL, "dh0_re/dh0_im must both be given");
  if (dh0_re && !h0_re) return fail(SPARC_EINVAL, "dh0 requested without h0");
  if (cplx && y_re && !y_im && !relu) return fail(SPARC_EINVAL, "y_im is required with y_re");
  const bool saved = y_re && !relu;  // y = h (rounded to the I/O dtype) only without the relu epilogue
  const void* ptrs[] = {w_re, w_im, dy_re, relu ? nullptr : dy_im, dw_re, dw_im,
                        saved ? y_re : nullptr, saved ? y_im : nullptr};
  if (sparc_status s = check_io_ptrs(d, pl, ptrs, 8)) return s;
  if (pl.gm == sparc::GATE_MODE) {
    const void* gp[] = {gate0, gate1, dgate0, dgate1};
    if (sparc_status s = check_gate_ptrs(d, pl, gp, 4)) return s;
  }
  if (saved) {  // P1 from the saved states: the fused kernels, when they apply
    const void* fp[] = {y_re, y_im, dy_re, dy_im, dw_re, dw_im, h0_re, h0_im, dh0_re, dh0_im};
    if (p1_fused_route(d, 1, fp, 10, chunk_state, workspace_bytes))
      return sparc::p1_fused_backward(d, static_cast<const float*>(gate0), static_cast<const float*>(gate1), nu_log,
                                      theta_log, y_re, y_im, h0_re, h0_im, segment_pos, dy_re, dy_im, dlast_re,
                                      dlast_im, dw_re, dw_im, static_cast<float*>(dgate0),
                                      static_cast<float*>(dgate1), dnu_log, dtheta_log, dh0_re, dh0_im, workspace,
                                      workspace_bytes, stream);
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (!pl.chain)
    if (sparc_status s = clear_ws(pl, workspace, st)) return s;
  sparc::ScanArgs a{};
  a.B = static_cast<int>(d->batch);
  a.T = static_cast<int>(d->length);
  a.M = static_cast<int>(d->modes);
  a.G = static_cast<int>(d->groups);
  a.gs = static_cast<int>(d->modes / d->groups);
  a.n_chunks = pl.n_chunks;
  a.n_mblocks = pl.n_mblocks;
  a.n_chains = pl.n_chains;
  a.flags = static_cast<uint32_t>(d->flags);
  a.spin_limit = g_wait_limit.load(std::memory_order_relaxed);
  a.g0 = gate0; a.g1 = gate1; a.nu_log = nu_log; a.theta_log = theta_log;
  a.w_re = w_re; a.w_im = w_im; a.h0_re = h0_re; a.h0_im = h0_im; a.segpos = segment_pos;
  a.chunk_state_in = chunk_state;
  a.dy_re = dy_re; a.dy_im = dy_im; a.dlast_re = dlast_re; a.dlast_im = dlast_im;
  a.dw_re = dw_re; a.dw_im = dw_im; a.dg0 = dgate0; a.dg1 = dgate1;
  a.dh0_re = dh0_re; a.dh0_im = dh0_im;
  if (saved) {
    a.y_re = const_cast<void*>(y_re);
    a.y_im = const_cast<void*>(y_im);
  }
  fill_ws(a, pl, workspace);
  if (!(saved && launch(2, d, pl, st, a)) && !launch(1, d, pl, st, a))
    return fail(SPARC_EUNSUPPORTED, "no backward kernel for this plan");
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(SPARC_EHIP, "scan backward launch: %s", hipGetErrorString(e));
  // deterministic reductions of the per-tile partials
  const int64_t rows = d->batch * d->length;
  if (pl.gm == sparc::GATE_CROSS) {
    const int per = pl.n_mblocks / static_cast<int>(d->groups);
    const int64_t n = rows * d->groups;
    const dim3 g(static_cast<unsigned>((n + 255) / 256));
    if (d->gate_dtype == SPARC_BF16) {
      hipLaunchKernelGGL(sparc::reduce_groups_kernel<sparc::bf16>, g, dim3(256), 0, st, a.part_g0, rows, pl.n_mblocks, static_cast<int>(d->groups), per, dgate0);
      if (cplx) hipLaunchKernelGGL(sparc::reduce_groups_kernel<sparc::bf16>, g, dim3(256), 0, st, a.part_g1, rows, pl.n_mblocks, static_cast<int>(d->groups), per, dgate1);
    } else {
      hipLaunchKernelGGL(sparc::reduce_groups_kernel<float>, g, dim3(256), 0, st, a.part_g0, rows, pl.n_mblocks, static_cast<int>(d->groups), per, dgate0);
      if (cplx) hipLaunchKernelGGL(sparc::reduce_groups_kernel<float>, g, dim3(256), 0, st, a.part_g1, rows, pl.n_mblocks, static_cast<int>(d->groups), per, dgate1);
    }
  }
  if (p1) {
    // one partial row per tile (look-back) or per batch row (chain)
    const int64_t prow = pl.chain ? d->batch : d->batch * pl.n_chunks;
    const float* in[2] = {a.part_nu, a.part_theta};
    float* out[2] = {dnu_log, dtheta_log};
    if (sparc_status s = sparc::column_sums(prow, d->modes, 2, in, out, stream)) return s;
  }
  e = hipGetLastError();
  if (e != hipSuccess) return fail(SPARC_EHIP, "scan backward reductions: %s", hipGetErrorString(e));
  return SPARC_OK;
}

uint32_t sparc_set_wait_limit(uint32_t polls) {
  return g_wait_limit.exchange(polls, std::memory_order_relaxed);
}

int sparc_scan_workspace_error(const void* workspace, sparc_stream_t stream) {
  uint32_t err = 0;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (hipMemcpyAsync(&err, static_cast<const uint32_t*>(workspace) + 1, 4, hipMemcpyDeviceToHost, st) != hipSuccess) return -1;
  if (hipStreamSynchronize(st) != hipSuccess) return -1;
  return err ? 1 : 0;
}

}  // extern "C"
#endif  // SPARC_SCAN_OWNS(0)
