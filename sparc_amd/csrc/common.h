// Device helpers shared by the SPARC HIP kernels (gfx950 / CDNA4).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sparc {

// ---------------------------------------------------------------------------
// element types
// ---------------------------------------------------------------------------
struct bf16 {  // storage tag: raw IEEE bfloat16 bits
  uint16_t bits;
};

__device__ __forceinline__ float bf16_bits_to_float(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// Round-to-nearest-even fp32 -> bf16 (v_cvt_pk_bf16_f32 on gfx950), two at a time.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;
  typedef __attribute__((__vector_size__(2 * sizeof(float)))) float float2_t;
  float2_t f = {lo, hi};
  bf16x2_t b = __builtin_convertvector(f, bf16x2_t);
  return __builtin_bit_cast(uint32_t, b);
}
__device__ __forceinline__ uint16_t pack_bf16(float v) {
  return (uint16_t)(pack_bf16x2(v, 0.0f) & 0xffffu);
}
// Both values rounded to bf16 (nearest even) and widened back to fp32.
__device__ __forceinline__ void round_bf16x2(float& a, float& b) {
  const uint32_t u = pack_bf16x2(a, b);
  a = __uint_as_float(u << 16);
  b = __uint_as_float(u & 0xffff0000u);
}

// transitions (values of sparc_transition)
enum Transition : int { TR_P1 = 0, TR_POLAR = 1, TR_CART = 2, TR_REAL = 3 };
// Kernel template argument TR = transition | TR_G32: TR_G32 marks fp32 gates
// beside bf16 I/O for the polar, cartesian and real transitions (the
// reference's generic scans load `a` in its own dtype, independently of the
// writes).  P1 gates are always fp32.
constexpr int TR_G32 = 4;
constexpr int tr_kind(int tr) { return tr & 3; }
constexpr bool tr_g32(int tr) { return (tr & TR_G32) != 0; }

// Raw vector of V elements of type IO, loaded/stored with one instruction.
template <typename IO, int V> struct Raw;
template <> struct Raw<bf16, 1> { using T = uint16_t; };
template <> struct Raw<bf16, 2> { using T = uint32_t; };
template <> struct Raw<bf16, 4> { using T = uint2; };
template <> struct Raw<bf16, 8> { using T = uint4; };
template <> struct Raw<float, 1> { using T = float; };
template <> struct Raw<float, 2> { using T = float2; };
template <> struct Raw<float, 4> { using T = float4; };

template <typename IO, int V>
__device__ __forceinline__ typename Raw<IO, V>::T load_raw(const void* base, int64_t index) {
  using R = typename Raw<IO, V>::T;
  return reinterpret_cast<const R*>(static_cast<const IO*>(base) + index)[0];
}
template <typename IO, int V>
__device__ __forceinline__ void store_raw(void* base, int64_t index, typename Raw<IO, V>::T v) {
  using R = typename Raw<IO, V>::T;
  reinterpret_cast<R*>(static_cast<IO*>(base) + index)[0] = v;
}

// Non-temporal variants: streamed data that is touched once per kernel (the
// nt cache hint: do not keep it in the caches ahead of data that is reused).
template <int NB> struct NtBits;
template <> struct NtBits<2> { using T = unsigned short; };
template <> struct NtBits<4> { using T = unsigned int; };
template <> struct NtBits<8> { typedef unsigned int T __attribute__((ext_vector_type(2))); };
template <> struct NtBits<16> { typedef unsigned int T __attribute__((ext_vector_type(4))); };

template <typename IO, int V>
__device__ __forceinline__ typename Raw<IO, V>::T load_raw_nt(const void* base, int64_t index) {
  using R = typename Raw<IO, V>::T;
  using N = typename NtBits<sizeof(R)>::T;
  const N n = __builtin_nontemporal_load(reinterpret_cast<const N*>(static_cast<const IO*>(base) + index));
  R r;
  __builtin_memcpy(&r, &n, sizeof(R));
  return r;
}
template <typename IO, int V>
__device__ __forceinline__ void store_raw_nt(void* base, int64_t index, typename Raw<IO, V>::T v) {
  using R = typename Raw<IO, V>::T;
  using N = typename NtBits<sizeof(R)>::T;
  N n;
  __builtin_memcpy(&n, &v, sizeof(R));
  __builtin_nontemporal_store(n, reinterpret_cast<N*>(static_cast<IO*>(base) + index));
}

// Buffer loads and stores with an explicit cache policy (the cpol immediate of
// gfx950 vector memory instructions: sc0 = 1, nt = 2, sc1 = 16).  sc1 on data
// that is reused only by the next launch keeps it out of the per-XCD L2 and
// serves it from the memory-side Infinity Cache.  A resource covers ``bytes``
// from ``base``; accesses past it read 0 and drop stores.
enum : int { CPOL_DEFAULT = 0, CPOL_SC0 = 1, CPOL_NT = 2, CPOL_SC1 = 16 };
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), bytes,
                                           0x00020000);
}
template <int V, int CPOL>
__device__ __forceinline__ void buffer_load_f32(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, float (&o)[V]) {
  static_assert(V == 1 || V == 2 || V == 4, "1, 2 or 4 floats");
  if constexpr (V == 4) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, CPOL);
#pragma unroll
    for (int k = 0; k < 4; ++k) o[k] = __uint_as_float(v[k]);
  } else if constexpr (V == 2) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, byte_off, 0, CPOL);
    o[0] = __uint_as_float(v[0]);
    o[1] = __uint_as_float(v[1]);
  } else {
    o[0] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, CPOL));
  }
}
template <int V, int CPOL>
__device__ __forceinline__ void buffer_store_f32(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, const float (&i)[V]) {
  static_assert(V == 1 || V == 2 || V == 4, "1, 2 or 4 floats");
  if constexpr (V == 4) {
    typedef uint32_t u4 __attribute__((ext_vector_type(4)));
    const u4 v = {__float_as_uint(i[0]), __float_as_uint(i[1]), __float_as_uint(i[2]), __float_as_uint(i[3])};
    __builtin_amdgcn_raw_buffer_store_b128(v, r, byte_off, 0, CPOL);
  } else if constexpr (V == 2) {
    typedef uint32_t u2 __attribute__((ext_vector_type(2)));
    const u2 v = {__float_as_uint(i[0]), __float_as_uint(i[1])};
    __builtin_amdgcn_raw_buffer_store_b64(v, r, byte_off, 0, CPOL);
  } else {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(i[0]), r, byte_off, 0, CPOL);
  }
}

// s_waitcnt vmcnt(0): every vector memory operation of the wave has completed.
__device__ __forceinline__ void wait_vm_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// A raw T (2, 4, 8 or 16 bytes) through a buffer resource at the lane's
// byte offset voff plus a wave-uniform byte offset soff (an SGPR operand: no
// per-lane address arithmetic), with cache policy CPOL.
template <typename T, int CPOL>
__device__ __forceinline__ T buf_load(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  T out;
  if constexpr (sizeof(T) == 2) {
    const unsigned short v = __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, CPOL);
    __builtin_memcpy(&out, &v, 2);
  } else if constexpr (sizeof(T) == 4) {
    const uint32_t v = __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, CPOL);
    __builtin_memcpy(&out, &v, 4);
  } else if constexpr (sizeof(T) == 8) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, CPOL);
    __builtin_memcpy(&out, &v, 8);
  } else {
    static_assert(sizeof(T) == 16, "2, 4, 8 or 16 bytes");
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, CPOL);
    __builtin_memcpy(&out, &v, 16);
  }
  return out;
}
template <typename T, int CPOL>
__device__ __forceinline__ void buf_store(T x, __amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  if constexpr (sizeof(T) == 2) {
    unsigned short v;
    __builtin_memcpy(&v, &x, 2);
    __builtin_amdgcn_raw_buffer_store_b16(v, r, voff, soff, CPOL);
  } else if constexpr (sizeof(T) == 4) {
    uint32_t v;
    __builtin_memcpy(&v, &x, 4);
    __builtin_amdgcn_raw_buffer_store_b32(v, r, voff, soff, CPOL);
  } else if constexpr (sizeof(T) == 8) {
    typedef uint32_t u2 __attribute__((ext_vector_type(2)));
    u2 v;
    __builtin_memcpy(&v, &x, 8);
    __builtin_amdgcn_raw_buffer_store_b64(v, r, voff, soff, CPOL);
  } else {
    // A store of more than 8 bytes reads its data registers after it issues:
    // a VALU write to them right behind it needs wait states.  The compiler
    // inserts them only for stores without a register soffset, and on gfx950
    // a 16-byte buffer store with an SGPR soffset measurably stored the
    // next step's value into its first dword now and then (the wide P1
    // backward in fp32, before this).  So the uniform offset joins the lane
    // offset (one add; the sum stays below 2^32 and past the resource for
    // dropped lanes) and soffset is the constant 0.
    static_assert(sizeof(T) == 16, "2, 4, 8 or 16 bytes");
    typedef uint32_t u4 __attribute__((ext_vector_type(4)));
    u4 v;
    __builtin_memcpy(&v, &x, 16);
    __builtin_amdgcn_raw_buffer_store_b128(v, r, voff + soff, 0, CPOL);
  }
}

// A 64-bit value every lane of the wave holds, moved to scalar registers, so
// that a memory instruction can take (kernel-argument pointer + this offset)
// as its scalar base and the lane's byte offset as its vector offset.
__device__ __forceinline__ int64_t wave_uniform(int64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(static_cast<uint64_t>(v) >> 32));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

template <typename T>
__device__ __forceinline__ T ldb(const void* base, int64_t byte_off, uint32_t lane_bytes) {
  return *reinterpret_cast<const T*>(static_cast<const char*>(base) + byte_off + lane_bytes);
}
template <typename T>
__device__ __forceinline__ void stb(void* base, int64_t byte_off, uint32_t lane_bytes, T v) {
  *reinterpret_cast<T*>(static_cast<char*>(base) + byte_off + lane_bytes) = v;
}
// Non-temporal forms of ldb / stb for streamed planes, each element of which is
// read or written once per launch: the nt cache policy keeps them from
// displacing lines that are reused.
template <typename T, bool NT = true>
__device__ __forceinline__ T ldn(const void* base, int64_t byte_off, uint32_t lane_bytes) {
  if constexpr (!NT) return ldb<T>(base, byte_off, lane_bytes);
  using N = typename NtBits<sizeof(T)>::T;
  const N n = __builtin_nontemporal_load(
      reinterpret_cast<const N*>(static_cast<const char*>(base) + byte_off + lane_bytes));
  T r;
  __builtin_memcpy(&r, &n, sizeof(T));
  return r;
}
template <typename T, bool NT = true>
__device__ __forceinline__ void stn(void* base, int64_t byte_off, uint32_t lane_bytes, T v) {
  if constexpr (!NT) { stb<T>(base, byte_off, lane_bytes, v); return; }
  using N = typename NtBits<sizeof(T)>::T;
  N n;
  __builtin_memcpy(&n, &v, sizeof(T));
  __builtin_nontemporal_store(n, reinterpret_cast<N*>(static_cast<char*>(base) + byte_off + lane_bytes));
}

template <typename IO, int V>
__device__ __forceinline__ void unpack(const typename Raw<IO, V>::T& r, float (&o)[V]) {
  if constexpr (sizeof(IO) == 4) {
    const float* f = reinterpret_cast<const float*>(&r);
#pragma unroll
    for (int v = 0; v < V; ++v) o[v] = f[v];
  } else if constexpr (V == 1) {
    o[0] = bf16_bits_to_float(r);
  } else {
    const uint32_t* w = reinterpret_cast<const uint32_t*>(&r);
#pragma unroll
    for (int v = 0; v < V / 2; ++v) {
      o[2 * v] = __uint_as_float(w[v] << 16);
      o[2 * v + 1] = __uint_as_float(w[v] & 0xffff0000u);
    }
  }
}

template <typename IO, int V>
__device__ __forceinline__ typename Raw<IO, V>::T pack(const float (&i)[V]) {
  typename Raw<IO, V>::T r;
  if constexpr (sizeof(IO) == 4) {
    float* f = reinterpret_cast<float*>(&r);
#pragma unroll
    for (int v = 0; v < V; ++v) f[v] = i[v];
  } else if constexpr (V == 1) {
    r = pack_bf16(i[0]);
  } else {
    uint32_t* w = reinterpret_cast<uint32_t*>(&r);
#pragma unroll
    for (int v = 0; v < V / 2; ++v) w[v] = pack_bf16x2(i[2 * v], i[2 * v + 1]);
  }
  return r;
}

template <typename IO>
__device__ __forceinline__ float load1(const void* base, int64_t index) {
  if constexpr (sizeof(IO) == 4) return static_cast<const float*>(base)[index];
  else return bf16_bits_to_float(static_cast<const uint16_t*>(base)[index]);
}
template <typename IO>
__device__ __forceinline__ float load1_nt(const void* base, int64_t index) {
  if constexpr (sizeof(IO) == 4) return __builtin_nontemporal_load(static_cast<const float*>(base) + index);
  else return bf16_bits_to_float(__builtin_nontemporal_load(static_cast<const uint16_t*>(base) + index));
}
template <typename IO>
__device__ __forceinline__ void store1(void* base, int64_t index, float v) {
  if constexpr (sizeof(IO) == 4) static_cast<float*>(base)[index] = v;
  else static_cast<uint16_t*>(base)[index] = pack_bf16(v);
}

// ---------------------------------------------------------------------------
// math
// ---------------------------------------------------------------------------
// Workgroups of a launch are handed to the 8 XCDs round-robin (workgroup i
// runs on XCD i % 8), and each XCD has its own L2.  Renumber workgroups so
// that consecutive work items (here: neighbouring mode blocks of one batch
// row, which share the 128-byte cache lines of their gates) run on the same
// XCD: XCD x takes items [x*per + min(x, rem), ...) in dispatch order.  A
// bijection on [0, n) for any n.
__device__ __forceinline__ int xcd_swizzle(int bid, int n) {
  constexpr int kXcds = 8;
  const int per = n / kXcds, rem = n % kXcds;
  const int x = bid % kXcds, k = bid / kXcds;
  return x * per + (x < rem ? x : rem) + k;
}

// exp(x) through the hardware base-2 exponential (v_exp_f32).
__device__ __forceinline__ float fast_exp(float x) {
  return __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
}

// theta = exp(theta_log) and its cosine and sine (returned in c, s), each
// evaluated in fp64 and rounded once to fp32.  A P1 transition turns the state
// by theta plus a small gate-dependent angle at every step, so an error in
// these per-mode constants is the same at every step and adds up over as many
// steps as a mode remembers (about 1 / (1 - |a|), tens of thousands of steps
// for slow modes).  fp32 evaluation (exp, then sincos of the rounded theta)
// leaves a few ulps: about 1e-4 relative error after 2k steps of a slow mode,
// against about 1e-5 with these constants.
__device__ inline float theta_rotation(float theta_log, float& c, float& s) {
  const double th = exp(static_cast<double>(theta_log));
  double sd, cd;
  sincos(th, &sd, &cd);
  c = static_cast<float>(cd);
  s = static_cast<float>(sd);
  return static_cast<float>(th);
}

// theta's cosine and sine as unevaluated fp32 sums hi + lo: hi is the fp64
// value rounded to fp32 (what theta_rotation returns) and lo the remainder,
// rounded.  Rotating by (hi + lo) removes the per-mode rounding of the
// constants themselves, which is the same at every step: over 8k steps of a
// slow mode it leaves about 1e-4 relative error with hi alone and under 1e-5
// with the pair.  The single-step kernels use it (they are bound by memory,
// so the two extra FMAs per rotation cost nothing there).
__device__ inline void theta_rotation_split(float theta_log, float& c, float& s, float& c_lo,
                                            float& s_lo) {
  const double th = exp(static_cast<double>(theta_log));
  double sd, cd;
  sincos(th, &sd, &cd);
  c = static_cast<float>(cd);
  s = static_cast<float>(sd);
  c_lo = static_cast<float>(cd - static_cast<double>(c));
  s_lo = static_cast<float>(sd - static_cast<double>(s));
}

// (c + c_lo + i (s + s_lo)) (cd + i sd) with the small products added first,
// so the result is rounded once
__device__ __forceinline__ void rotate_split(float c, float s, float c_lo, float s_lo, float cd,
                                             float sd, float& re, float& im) {
  const float lo_r = fmaf(c_lo, cd, -s_lo * sd);
  const float lo_i = fmaf(s_lo, cd, c_lo * sd);
  re = fmaf(c, cd, fmaf(-s, sd, lo_r));
  im = fmaf(s, cd, fmaf(c, sd, lo_i));
}

// sin and cos of |x| <= pi/4 by their Taylor series (truncation error below
// 1e-9 on that interval, i.e. well under one fp32 ulp of the result).
__device__ __forceinline__ void sincos_quarter(float x, float& s, float& c) {
  const float x2 = x * x;
  // sin x = x (1 - x^2/3! + x^4/5! - x^6/7! + x^8/9!)
  float ps = 2.7557319223985893e-6f;          // 1/9!
  ps = fmaf(ps, x2, -1.9841269841269841e-4f); // 1/7!
  ps = fmaf(ps, x2, 8.3333333333333332e-3f);  // 1/5!
  ps = fmaf(ps, x2, -1.6666666666666666e-1f); // 1/3!
  s = fmaf(ps * x2, x, x);
  // cos x = 1 - x^2/2! + x^4/4! - x^6/6! + x^8/8! - x^10/10!
  float pc = -2.7557319223985888e-7f;         // 1/10!
  pc = fmaf(pc, x2, 2.4801587301587302e-5f);  // 1/8!
  pc = fmaf(pc, x2, -1.3888888888888889e-3f); // 1/6!
  pc = fmaf(pc, x2, 4.1666666666666664e-2f);  // 1/4!
  pc = fmaf(pc, x2, -0.5f);
  c = fmaf(pc, x2, 1.0f);
}

// expm1(x) for x <= 0: the Taylor series to x^4/4! for |x| < 1/16 (relative
// error < 1.3e-7, about one fp32 ulp), exp(x) - 1 beyond (relative error
// < 1e-6: no cancellation left to amplify the exponential's rounding)
__device__ __forceinline__ float expm1_nonpos(float x) {
  float p = 1.0f / 24.0f;
  p = fmaf(p, x, 1.0f / 6.0f);
  p = fmaf(p, x, 0.5f);
  p = fmaf(p, x, 1.0f);
  p *= x;
  return x > -0.0625f ? p : fast_exp(x) - 1.0f;
}

// sin and cos of |u| <= pi/2 by minimax polynomials, sin u = u + u^3 P(u^2)
// (P of degree 3) and cos u = 1 + u^2 Q(u^2) (Q of degree 4).  The
// coefficients minimise the maximum relative error of sin and the absolute
// error of cos on [0, pi/2] (Lawson's iteratively reweighted least squares);
// evaluated in fp32 both stay within 1.2e-7 of the true values, the same as
// the Taylor series to u^11 / u^12 they replace, with two fewer FMAs.
__device__ __forceinline__ void sincos_half(float u, float& s, float& c) {
  const float u2 = u * u;
  float ps = 2.6057807644974673e-6f;
  ps = fmaf(ps, u2, -1.9809603691101074e-4f);
  ps = fmaf(ps, u2, 8.33306647837162e-3f);
  ps = fmaf(ps, u2, -1.6666659712791443e-1f);
  s = fmaf(ps * u2, u, u);
  float pc = -2.607710598567792e-7f;
  pc = fmaf(pc, u2, 2.4761886379565112e-5f);
  pc = fmaf(pc, u2, -1.38884037733078e-3f);
  pc = fmaf(pc, u2, 4.166664183139801e-2f);
  pc = fmaf(pc, u2, -0.5f);
  c = fmaf(pc, u2, 1.0f);
}

// expm1_nonpos and sincos_half over N independent arguments, written one
// polynomial level at a time across all N: the N dependency chains then
// interleave in the instruction stream (the compiler keeps this order), so
// a wave has independent work between dependent instructions.
template <int N>
__device__ __forceinline__ void expm1_nonpos_n(const float (&x)[N], float (&o)[N]) {
  float p[N], e[N];
#pragma unroll
  for (int i = 0; i < N; ++i) p[i] = fmaf(1.0f / 24.0f, x[i], 1.0f / 6.0f);
#pragma unroll
  for (int i = 0; i < N; ++i) e[i] = __builtin_amdgcn_exp2f(x[i] * 1.4426950408889634f);
#pragma unroll
  for (int i = 0; i < N; ++i) p[i] = fmaf(p[i], x[i], 0.5f);
#pragma unroll
  for (int i = 0; i < N; ++i) p[i] = fmaf(p[i], x[i], 1.0f);
#pragma unroll
  for (int i = 0; i < N; ++i) p[i] *= x[i];
#pragma unroll
  for (int i = 0; i < N; ++i) o[i] = x[i] > -0.0625f ? p[i] : e[i] - 1.0f;
}
template <int N>
__device__ __forceinline__ void sincos_half_n(const float (&u)[N], float (&s)[N], float (&c)[N]) {
  float u2[N], ps[N], pc[N];
#pragma unroll
  for (int i = 0; i < N; ++i) u2[i] = u[i] * u[i];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    ps[i] = fmaf(2.6057807644974673e-6f, u2[i], -1.9809603691101074e-4f);
    pc[i] = fmaf(-2.607710598567792e-7f, u2[i], 2.4761886379565112e-5f);
  }
#pragma unroll
  for (int i = 0; i < N; ++i) {
    ps[i] = fmaf(ps[i], u2[i], 8.33306647837162e-3f);
    pc[i] = fmaf(pc[i], u2[i], -1.38884037733078e-3f);
  }
#pragma unroll
  for (int i = 0; i < N; ++i) {
    ps[i] = fmaf(ps[i], u2[i], -1.6666659712791443e-1f);
    pc[i] = fmaf(pc[i], u2[i], 4.166664183139801e-2f);
  }
#pragma unroll
  for (int i = 0; i < N; ++i) {
    s[i] = fmaf(ps[i] * u2[i], u[i], u[i]);
    pc[i] = fmaf(pc[i], u2[i], -0.5f);
  }
#pragma unroll
  for (int i = 0; i < N; ++i) c[i] = fmaf(pc[i], u2[i], 1.0f);
}

// sin and cos of 2 pi r through the hardware (v_sin_f32, v_cos_f32 take the
// angle in revolutions).  Measured on MI355X over |2 pi r| <= pi/2 against
// fp64: max abs error 1.4e-7 (sin) and 1.7e-7 (cos), mean error below 1e-8
// (no bias that adds up over steps); each instruction issues at about half the
// FMA rate, against 6 FMAs per function for the polynomials above.  Used for
// bf16 I/O only: fp32 I/O keeps sincos_half (1.3e-7 / 0.9e-7, about 1 ulp).
__device__ __forceinline__ void sincos_rev_hw(float r, float& s, float& c) {
  s = __builtin_amdgcn_sinf(r);
  c = __builtin_amdgcn_cosf(r);
}
constexpr float kNegInv2Pi = -0.15915494309189535f;  // -1 / (2 pi): a phase in radians -> revolutions, negated

// Keeps the compiler from moving this wave's LDS accesses across it.  A
// wave's own LDS reads and writes are performed in issue order, so a value
// one lane writes is seen by a later read of another lane of the same wave
// without a workgroup barrier (which would also wait for every outstanding
// global load); no instruction is emitted.
__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ---------------------------------------------------------------------------
// cross-lane moves (every lane of the wave must be active: a DPP read from an
// inactive lane returns 0)
// ---------------------------------------------------------------------------
// A DPP move of src with the given control; lanes outside BANKS (4-lane
// banks of each 16-lane row, bit b = lanes 4b..4b+3) keep old.
template <int CTRL, int BANKS = 0xF>
__device__ __forceinline__ float dpp_mov(float old, float src) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(src), CTRL, 0xF, BANKS,
                                                    BANKS == 0xF));
}
constexpr int kDppIdentity = 0xE4;     // quad_perm [0, 1, 2, 3]
constexpr int kDppXor1 = 0xB1;         // quad_perm [1, 0, 3, 2]: lane ^ 1
constexpr int kDppXor2 = 0x4E;         // quad_perm [2, 3, 0, 1]: lane ^ 2
constexpr int kDppRowShl = 0x100;      // + n: lane i reads lane i + n of its row
constexpr int kDppRowShr = 0x110;      // + n: lane i reads lane i - n of its row
constexpr int kDppRowRor = 0x120;      // + n: lane i reads lane (i - n) mod 16 of its row
constexpr int kDppRowMirror = 0x140;   // lane i reads lane 15 - i of its row
constexpr int kDppHalfMirror = 0x141;  // lane i reads lane 7 - i of its half-row

// x[l] + x[l ^ 16] (PAIR 16) or x[l] + x[l ^ 32] (PAIR 32) in every lane: a
// swap of the register's row halves with itself (v_permlane16_swap /
// v_permlane32_swap), no LDS.
template <int PAIR>
__device__ __forceinline__ float pair_sum(float x) {
  const uint32_t u = __float_as_uint(x);
  if constexpr (PAIR == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  } else {
    static_assert(PAIR == 32, "16 or 32");
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
}

// Sum over aligned groups of lpg lanes (a power of two up to 64, wave-
// uniform), in every lane of the group.
__device__ __forceinline__ float group_sum(float x, int lpg) {
  if (lpg >= 2) x += dpp_mov<kDppXor1>(0.0f, x);
  if (lpg >= 4) x += dpp_mov<kDppXor2>(0.0f, x);
  if (lpg >= 8) x += dpp_mov<kDppHalfMirror>(0.0f, x);  // the other quad of the 8 lanes
  if (lpg >= 16) x += dpp_mov<kDppRowMirror>(0.0f, x);  // the other half of the row
  if (lpg >= 32) x = pair_sum<16>(x);
  if (lpg >= 64) x = pair_sum<32>(x);
  return x;
}

// ---------------------------------------------------------------------------
// wave reductions of several values per lane
// ---------------------------------------------------------------------------
// N values per lane -> the wave sums of all N (a reduce-scatter butterfly:
// each stage exchanges half of the values with the lane 32, 16, 8 or 4 away
// and keeps the other half).  The 32- and 16-lane stages swap register
// halves (v_permlane32_swap / v_permlane16_swap: one swap and one add per
// pair, no selects); the 8- and 4-lane stages choose what to keep and send
// with bank-masked DPP moves and read the partner through DPP, so nothing
// goes through LDS and no value is selected by a lane-dependent index.  The
// rest of each group of lanes is summed into its first lane.  On return the
// lanes l with l % G == 0 hold in v[0..K-1] the sums of values
// (l / G) * K ... (l / G) * K + K - 1, with K = max(1, N / 16) and
// G = 64 K / N; the other lanes hold partial sums.  Fixed order: the result
// does not depend on timing.
template <int N>
__device__ __forceinline__ void wave_sums_to_leaders(float (&v)[N]) {
  static_assert(N == 4 || N == 8 || N == 16 || N == 32, "4, 8, 16 or 32 values per lane");
#pragma unroll
  for (int i = 0; i < N / 2; ++i) {  // lanes 32 apart: the lower half of the wave keeps values 0 .. N/2-1
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[i]), __float_as_uint(v[i + N / 2]), false, false);
    v[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
#pragma unroll
  for (int i = 0; i < N / 4; ++i) {  // lanes 16 apart: even rows keep the lower half
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[i]), __float_as_uint(v[i + N / 4]), false, false);
    v[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  if constexpr (N >= 8) {
#pragma unroll
    for (int i = 0; i < N / 8; ++i) {  // lanes 8 apart: lanes 8-15 of a row (banks 2, 3) keep the upper half
      const float keep = dpp_mov<kDppIdentity, 0xC>(v[i], v[i + N / 8]);
      const float send = dpp_mov<kDppIdentity, 0xC>(v[i + N / 8], v[i]);
      v[i] = keep + dpp_mov<kDppRowRor + 8>(0.0f, send);  // lane ^ 8
    }
  }
  if constexpr (N >= 16) {
#pragma unroll
    for (int i = 0; i < N / 16; ++i) {  // lanes 4 apart: banks 1, 3 keep the upper half
      const float keep = dpp_mov<kDppIdentity, 0xA>(v[i], v[i + N / 16]);
      const float send = dpp_mov<kDppIdentity, 0xA>(v[i + N / 16], v[i]);
      float recv = dpp_mov<kDppRowShr + 4, 0xA>(0.0f, send);  // banks 1, 3 read lane - 4
      recv = dpp_mov<kDppRowShl + 4, 0x5>(recv, send);        // banks 0, 2 read lane + 4
      v[i] = keep + recv;
    }
  }
  constexpr int K = N >= 16 ? N / 16 : 1;
  constexpr int G = 64 * K / N;  // lanes per group, within one row
#pragma unroll
  for (int k = 0; k < K; ++k) {
    if constexpr (G >= 16) v[k] += dpp_mov<kDppRowShl + 8>(0.0f, v[k]);
    if constexpr (G >= 8) v[k] += dpp_mov<kDppRowShl + 4>(0.0f, v[k]);
    if constexpr (G >= 4) v[k] += dpp_mov<kDppRowShl + 2>(0.0f, v[k]);
    if constexpr (G >= 2) v[k] += dpp_mov<kDppRowShl + 1>(0.0f, v[k]);
  }
}

// relu that keeps NaN, as torch.relu does (fmaxf(NaN, 0) is 0)
__device__ __forceinline__ float relu_keep_nan(float v) { return v > 0.0f ? v : (v != v ? v : 0.0f); }

// tanh(x) = 1 - 2 / (1 + e^{2x}) through one hardware exponential and
// reciprocal (absolute error ~1e-7; saturates to +-1 through e^{2x} = inf / 0)
__device__ __forceinline__ float tanh_fast(float x) {
  const float e = __builtin_amdgcn_exp2f(x * 2.8853900817779268f);  // 2 log2(e)
  return fmaf(-2.0f, __builtin_amdgcn_rcpf(1.0f + e), 1.0f);
}

// sin and cos for moderate |x| (gate phases, a few multiples of pi):
// x = k*(pi/2) + r with a two-term Cody-Waite split of pi/2, then the quadrant
// k mod 4 selects sign and swap.
__device__ __forceinline__ void sincos_moderate(float x, float& s, float& c) {
  const float k = rintf(x * 0.63661977236758134f);  // 2/pi
  float r = fmaf(k, -1.5707963705062866f, x);        // pi/2 rounded to fp32
  r = fmaf(k, 4.3711388286737929e-8f, r);            // minus the rounding error of that constant
  float sr, cr;
  sincos_quarter(r, sr, cr);
  const int q = static_cast<int>(k) & 3;
  const float ss = (q & 1) ? cr : sr;
  const float cc = (q & 1) ? sr : cr;
  s = (q & 2) ? -ss : ss;
  c = ((q + 1) & 2) ? -cc : cc;
}

// ---------------------------------------------------------------------------
// cross-workgroup publication of chunk carries
// ---------------------------------------------------------------------------
// Carries travel between workgroups that may sit on different XCDs, whose L2
// caches are not coherent with each other.  Every value a consumer reads is
// written with an agent-scope store (the sc1 cache policy: written through to
// the device coherence point) and read with an agent-scope load (sc1: not
// served from a possibly stale L2 line).  The producer waits for its own
// stores to complete (s_waitcnt vmcnt(0)) before it stores the flag, so a
// consumer that has observed the flag observes the data.  No L2 writeback or
// invalidate is needed for these few lines.
template <typename T>
__device__ __forceinline__ void store_agent(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ T load_agent(const T* p) {
  return __hip_atomic_load(const_cast<T*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void wait_stores_complete() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0), expcnt/lgkmcnt untouched (gfx9 encoding)
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

enum : uint32_t { FLAG_EMPTY = 0, FLAG_AGGREGATE = 1, FLAG_INCLUSIVE = 2 };


}  // namespace sparc

// ---------------------------------------------------------------------------
// host-side error reporting shared by every translation unit of the library
// ---------------------------------------------------------------------------
#include <stdarg.h>
#include <stdio.h>
namespace sparc {
inline char* error_buffer() {
  static thread_local char buf[512] = "";
  return buf;
}
// The bound on each cross-workgroup wait, in polls (sparc_set_wait_limit).
uint32_t wait_limit();
}  // namespace sparc
