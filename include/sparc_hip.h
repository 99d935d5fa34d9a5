/*
 * sparc_hip.h -- C ABI of the MI355X (gfx950) SPARC scan library
 * (libsparc_hip.so).
 *
 * Plain pointers and sizes only.  Every tensor is caller-allocated device
 * memory, row-major and contiguous; every call is enqueued on the caller's
 * HIP stream and returns without synchronising (sparc_mixer_backward may also
 * fork work onto a library-owned stream and joins it back before it returns:
 * see there).  Scratch memory comes in
 * through ``workspace`` (size from the matching *_workspace_bytes query,
 * contents undefined on entry); calls that share one workspace must be
 * ordered on one stream.  No entry point allocates device memory.
 *
 * Shapes: B batch rows, T time steps, M complex modes (or M real channels for
 * the real scan), G gate groups per token with group size M/G (mode m uses
 * gate m / (M/G)).  The mode axis of a model with D channels of N states is
 * m = d*N + n, so G = D shares one gate pair across a channel's N states and
 * G = 1 is the reference module (one (eta, delta) pair per token).
 *
 * Errors: a non-zero sparc_status; sparc_last_error() describes the most
 * recent failure of the calling thread.
 */
#ifndef SPARC_HIP_H
#define SPARC_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* sparc_stream_t; /* a hipStream_t; NULL = default stream */

typedef enum sparc_status {
  SPARC_OK = 0,
  SPARC_EINVAL = 1,       /* bad shape, pointer, dtype or flag combination */
  SPARC_EUNSUPPORTED = 2, /* valid request this build does not implement */
  SPARC_EHIP = 3,         /* a HIP runtime call failed */
  SPARC_EWORKSPACE = 4    /* workspace missing or too small */
} sparc_status;

typedef enum sparc_dtype { SPARC_F32 = 0, SPARC_BF16 = 1 } sparc_dtype;

typedef enum sparc_transition {
  /* a = rho*exp(i*(theta_m + (1-rho)*delta)), rho = exp(-nu_m*exp(eta));
   * gate0 = eta, gate1 = delta (fp32), nu_m = exp(nu_log), theta_m = exp(theta_log).
   * sparc-kernal/forward/scan.py:941-946 (reference P1 transition) */
  SPARC_TRANSITION_P1 = 0,
  /* a = r*exp(i*phi); gate0 = r (retention), gate1 = phi (phase) */
  SPARC_TRANSITION_POLAR = 1,
  /* a = gate0 + i*gate1 (G = M is the reference's complex_scan) */
  SPARC_TRANSITION_CARTESIAN = 2,
  /* real scan h = a*h + b; gate0 = a (G = M is the reference's real scans);
   * w_im, y_im, gate1 and every imaginary pointer are NULL */
  SPARC_TRANSITION_REAL = 3
} sparc_transition;

enum {
  /* y is the module output relu(cat(h_re, h_im)) [B,T,2M] written through
   * y_re (y_im NULL); in the backward dy_re is the gradient of that output
   * (dy_im NULL).  Complex transitions only. */
  SPARC_FLAG_RELU_OUTPUT = 1,
  /* the transition of step 0 is replaced by 0 (drops h0).  A non-NULL
   * segment_pos takes precedence: steps with segment_pos[b,t] == 0 reset. */
  SPARC_FLAG_RESET_FIRST = 2,
  /* Algorithm selection (default: automatic from the shape).  LOOKBACK:
   * every (chain, chunk) tile is its own workgroup and chunk carries pass
   * between workgroups (decoupled look-back); parallel over T, for few
   * (batch row, mode block) chains.  CHAIN: one workgroup walks a whole
   * chain, carries stay on the CU; for many chains.  SERIAL: one wave walks
   * a whole chain step by step (no sub-chunk maps, no barriers); for gates
   * shared by the lanes of a group (polar, cartesian, real) and enough chains
   * to give every SIMD a wave; other shapes fall back to CHAIN.  Without a
   * flag, a P1 scan with G = 1 (resets included), M a multiple of 4 and
   * 8-byte aligned planes runs on the one-wave-per-chain fused
   * kernels of the module path (time segments for few chains); its backward
   * too when y_re/y_im are given without RELU_OUTPUT.  Same results up to
   * float rounding; the saved chunk states of any feed any backward. */
  SPARC_FLAG_ALGO_LOOKBACK = 4,
  SPARC_FLAG_ALGO_CHAIN = 8,
  SPARC_FLAG_ALGO_SERIAL = 16
};

typedef struct sparc_scan_desc {
  int64_t batch;      /* B */
  int64_t length;     /* T >= 0 */
  int64_t modes;      /* M */
  int64_t groups;     /* G, divides M */
  int32_t transition; /* sparc_transition */
  int32_t io_dtype;   /* sparc_dtype of w, y, dy, dw */
  int32_t gate_dtype; /* sparc_dtype of gate0/gate1/dgate*: F32 for P1; for the other
                       * transitions io_dtype, or F32 beside BF16 I/O (the reference's
                       * generic scans load `a` in its own dtype and upcast it:
                       * sparc-kernal/forward/scan.py:629-630, :707-710) */
  int32_t flags;      /* SPARC_FLAG_* */
} sparc_scan_desc;

/* Time steps per chunk (the granularity of saved chunk states) and the
 * number of chunks, ceil(T / chunk). */
int64_t sparc_scan_chunk_length(const sparc_scan_desc* d);
int64_t sparc_scan_chunk_count(const sparc_scan_desc* d);

/* Bytes of workspace needed by sparc_scan_forward (direction 0) or
 * sparc_scan_backward (direction 1). */
size_t sparc_scan_workspace_bytes(const sparc_scan_desc* d, int direction);

/*
 * Forward chunked scan: h_t = a_t h_{t-1} + w_t, fp32 state, one pass over
 * the inputs.  Replaces _SPARCChunkScan.forward
 * (sparc-kernal/backward/scan.py:1126-1372: _sparc_chunk_summary,
 * _sparc_chunk_prefix / hierarchical / grouped carries, _sparc_chunk_replay),
 * _RealChunkScan.forward (:825-860), _ComplexScan.forward (:887-904),
 * _SPARCScan / _SPARCTiledSerialScan forward (:922-1015) and the output
 * epilogue torch.cat((out_r, out_i), -1).relu() (forward/scan.py:1598-1603).
 *
 *   gate0, gate1   [B,T,G] gate_dtype
 *   nu_log, theta_log [M] fp32 (P1 only, else NULL)
 *   w_re, w_im     [B,T,M] io_dtype
 *   h0_re, h0_im   [B,M] fp32 initial state, or NULL for zero
 *   segment_pos    [B,T] int32 or NULL
 *   y_re, y_im     [B,T,M] io_dtype (or y_re = [B,T,2M] with RELU_OUTPUT)
 *   chunk_state    [B, n_chunks, M, 2] fp32 (real: [B, n_chunks, M]): the
 *                  state after the last step of every chunk.  Its last chunk
 *                  is the final state ("cache" of return_cache=True); the
 *                  backward reads it to recompute states.
 */
sparc_status sparc_scan_forward(const sparc_scan_desc* d,
                                const void* gate0, const void* gate1,
                                const float* nu_log, const float* theta_log,
                                const void* w_re, const void* w_im,
                                const float* h0_re, const float* h0_im,
                                const int32_t* segment_pos,
                                void* y_re, void* y_im,
                                float* chunk_state,
                                void* workspace, size_t workspace_bytes,
                                sparc_stream_t stream);

/*
 * Backward of sparc_scan_forward: reverse-time scan of the adjoint
 * lambda_{t-1} = conj(a_t) lambda_t + dy_{t-1}.  The states h_{t-1} that the
 * transition gradients need are either read from the forward's saved output
 * (y_re/y_im given, no RELU_OUTPUT: y is h rounded to the I/O dtype, the
 * states the reference's own backward uses, backward/scan.py:1325-1329), or
 * recomputed in fp32 from w and chunk_state (no [B,T,M] state is saved).
 * Replaces
 * _SPARCChunkScan.backward (sparc-kernal/backward/scan.py:1375-1640:
 * _sparc_reverse_chunk_summary / _prefix / _replay and
 * _reduce_shared_control_gradients, backward/control.py:139-152),
 * _RealChunkScan.backward (:862-884), _ComplexScan.backward (:906-919) and
 * _SPARCTiledSerialScan.backward (:1023-1070).  Gate and parameter
 * gradient reductions are deterministic (fixed-order partial sums, no float
 * atomics).
 *
 *   w_re, w_im, chunk_state   as given to / written by the forward (always
 *                  required: every plan can fall back to recomputing)
 *   y_re, y_im     [B,T,M] io_dtype: the forward's outputs, or NULL.  Ignored
 *                  with RELU_OUTPUT.  When given, plans with lane-shared gates
 *                  (polar, cartesian, real; chain-serial) read the states
 *                  from them instead of recomputing them; other plans ignore
 *                  them.
 *   dy_re, dy_im   [B,T,M] io_dtype (or dy_re = [B,T,2M] with RELU_OUTPUT)
 *   dlast_re/_im   [B,M] fp32 gradient of the final state, or NULL
 *   dw_re, dw_im   [B,T,M] io_dtype, written
 *   dgate0/dgate1  [B,T,G] gate_dtype, written
 *   dnu_log, dtheta_log [M] fp32 (P1 only), written (not accumulated)
 *   dh0_re/_im     [B,M] fp32, written when h0 was given (else NULL)
 */
sparc_status sparc_scan_backward(const sparc_scan_desc* d,
                                 const void* gate0, const void* gate1,
                                 const float* nu_log, const float* theta_log,
                                 const void* w_re, const void* w_im,
                                 const void* y_re, const void* y_im,
                                 const float* h0_re, const float* h0_im,
                                 const int32_t* segment_pos,
                                 const float* chunk_state,
                                 const void* dy_re, const void* dy_im,
                                 const float* dlast_re, const float* dlast_im,
                                 void* dw_re, void* dw_im,
                                 void* dgate0, void* dgate1,
                                 float* dnu_log, float* dtheta_log,
                                 float* dh0_re, float* dh0_im,
                                 void* workspace, size_t workspace_bytes,
                                 sparc_stream_t stream);

/* Host-synchronising check of a workspace after forward/backward calls: 0 if
 * no cross-workgroup wait exceeded its bound, else 1.  For tests. */
int sparc_scan_workspace_error(const void* workspace, sparc_stream_t stream);

/* The bound on each cross-workgroup wait of the look-back kernels and of the
 * one-launch module backward (sparc_mixer_backward), in polls (default 2^20,
 * about a second).  A wait that reaches it sets the workspace error word
 * (sparc_scan_workspace_error, which reads either workspace) and its
 * workgroup carries on, so every launch finishes; the results of such a
 * launch are invalid (NaN where they depend on the missing value).  Applies
 * to launches issued after the call, process-wide; returns the previous
 * bound.  For tests and diagnostics (0: every wait fails at once).  No
 * counterpart in the reference, whose Triton scans have no cross-workgroup
 * waits. */
uint32_t sparc_set_wait_limit(uint32_t polls);

/*
 * P1 write prologue w = gain * (tanh x_re + i tanh x_im) with
 * gain = exp(wlg) * sqrt(expm1(-2 nu e^eta) / expm1(-2 nu)) * 2 sigmoid(q),
 * q = (delta/(pi/2)) * wpr + (eta/log 16) * wrr.  rows = B*T.
 * Replaces _latest_write_forward (sparc-kernal/forward/control.py:166-195).
 *   x [rows, 2M] io_dtype; eta, delta [rows] fp32; nu_log, write_log_gain,
 *   write_phase_response, write_radial_response [M] fp32;
 *   w_re, w_im [rows, M] io_dtype.  With rows = 0 nothing is read or
 *   written and every pointer may be NULL.
 */
sparc_status sparc_write_forward(int64_t rows, int64_t modes, int32_t io_dtype,
                                 const void* x, const float* eta, const float* delta,
                                 const float* nu_log, const float* write_log_gain,
                                 const float* write_phase_response,
                                 const float* write_radial_response,
                                 void* w_re, void* w_im, sparc_stream_t stream);

size_t sparc_write_workspace_bytes(int64_t rows, int64_t modes);

/*
 * Backward of the write prologue.  Replaces _latest_write_backward
 * (sparc-kernal/backward/control.py:10-89) with deterministic reductions.
 *   dw_re, dw_im [rows, M] io_dtype; dx [rows, 2M] io_dtype (written);
 *   deta, ddelta [rows] fp32 (written); dnu_log, dwrite_log_gain,
 *   dwrite_phase_response, dwrite_radial_response [M] fp32 (written).
 *   With rows = 0 the parameter gradients are zeroed and the row tensors
 *   and the workspace may be NULL.
 */
sparc_status sparc_write_backward(int64_t rows, int64_t modes, int32_t io_dtype,
                                  const void* x, const float* eta, const float* delta,
                                  const float* nu_log, const float* write_log_gain,
                                  const float* write_phase_response,
                                  const float* write_radial_response,
                                  const void* dw_re, const void* dw_im,
                                  void* dx, float* deta, float* ddelta,
                                  float* dnu_log, float* dwrite_log_gain,
                                  float* dwrite_phase_response,
                                  float* dwrite_radial_response,
                                  void* workspace, size_t workspace_bytes,
                                  sparc_stream_t stream);

/*
 * One fused P1 decode step for B independent rows: controls (two dot
 * products over 2M), transition, write, state update, relu(cat) output.
 * Replaces _latest_sparc_decode / latest_sparc_decode
 * (sparc-kernal/forward/decode.py:10-75) and the eager step (:296-306).
 *   x [B, 2M] io_dtype; phase_direction, radial_direction [2M+1] fp32;
 *   nu_log, theta_log, write_log_gain, write_phase_response,
 *   write_radial_response [M] fp32; state_re/_im [B,M] fp32 (read);
 *   new_re/_im [B,M] fp32 (written; may alias state_re/_im for an in-place
 *   update: every element is read before it is written, by the same thread);
 *   y [B, 2M] io_dtype.
 */
sparc_status sparc_decode_step(int64_t batch, int64_t modes, int32_t io_dtype,
                               const void* x,
                               const float* phase_direction, const float* radial_direction,
                               const float* nu_log, const float* theta_log,
                               const float* write_log_gain,
                               const float* write_phase_response,
                               const float* write_radial_response,
                               const float* state_re, const float* state_im,
                               float* new_re, float* new_im, void* y,
                               sparc_stream_t stream);

/*
 * Prepared decode: the per-mode constants of the P1 step are computed once
 * (consts [M, 8] fp32: nu, cos theta, sin theta, 4 exp(2 write_log_gain) /
 * expm1(-2 nu), -log2(e) write_phase_response, -log2(e)
 * write_radial_response, and the fp64 remainders of cos theta and sin theta
 * as fp32) and reused by every step while the
 * parameters do not change.  The step runs the
 * two control dot products split over several workgroups per row (partials in
 * the workspace) and then the per-(row, mode) update.  Same semantics and
 * arguments as sparc_decode_step otherwise (sparc-kernal/forward/decode.py:
 * 10-75); modes must be a multiple of 4.  The reference recomputes every
 * per-mode quantity on each step (decode.py:37-47).
 */
size_t sparc_decode_workspace_bytes(int64_t batch, int64_t modes);
sparc_status sparc_decode_prepare(int64_t modes, const float* nu_log, const float* theta_log,
                                  const float* write_log_gain,
                                  const float* write_phase_response,
                                  const float* write_radial_response,
                                  float* consts, sparc_stream_t stream);
sparc_status sparc_decode_step_prepared(int64_t batch, int64_t modes, int32_t io_dtype,
                                        const void* x,
                                        const float* phase_direction,
                                        const float* radial_direction,
                                        const float* consts,
                                        const float* state_re, const float* state_im,
                                        float* new_re, float* new_im, void* y,
                                        void* workspace, size_t workspace_bytes,
                                        sparc_stream_t stream);

/*
 * sparc_decode_step_prepared without a workspace argument, for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid allocation).  No counterpart in the reference.  The
 * partial sums live in a library-owned device array of 512 KiB + 256 B per
 * GPU (batch <= 4096 rows; larger batches return SPARC_EINVAL), kept until
 * the process ends; nothing is allocated.  Every call on a GPU shares that
 * GPU's array: calls that overlap on one GPU (concurrent streams, threads)
 * race and must be ordered by the caller.  The stream must belong to the
 * current device.  Same arguments and results as sparc_decode_step_prepared.
 */
sparc_status sparc_decode_step_prepared_noalloc(int64_t batch, int64_t modes, int32_t io_dtype,
                                                const void* x,
                                                const float* phase_direction,
                                                const float* radial_direction,
                                                const float* consts,
                                                const float* state_re, const float* state_im,
                                                float* new_re, float* new_im, void* y,
                                                sparc_stream_t stream);

/*
 * One step of the scan for B independent rows, with the state carried by the
 * caller: h <- a h + w, fp32 state updated in place (the scan-core decode
 * step).  The same as sparc_scan_forward with T = 1 and h0 = state: the
 * reference's serial scan with an initial state at L = 1
 * (_sparc_tiled_serial_forward, sparc-kernal/forward/scan.py:806-854, as
 * called by sparc_scan_with_last, sparc-kernal/backward/scan.py:1857-1877).
 *   d             batch, modes, groups, transition, dtypes; flags RELU_OUTPUT
 *                 (y layout) and RESET_FIRST (a := 0); length is ignored
 *   gate0, gate1  [B,G] (fp32 eta, delta for P1)
 *   nu_log, theta_log [M] fp32 (P1 only)
 *   w_re, w_im    [B,M] io_dtype
 *   state_re/_im  [B,M] fp32, read and written
 *   y_re, y_im    [B,M] io_dtype copy of the new state (or y_re = relu(cat)
 *                 [B,2M] with RELU_OUTPUT), or NULL for none
 */
sparc_status sparc_scan_step(const sparc_scan_desc* d,
                             const void* gate0, const void* gate1,
                             const float* nu_log, const float* theta_log,
                             const void* w_re, const void* w_im,
                             float* state_re, float* state_im,
                             void* y_re, void* y_im,
                             sparc_stream_t stream);

/*
 * Deterministic sum over rows of a [rows, cols] fp32 matrix into [cols]
 * (or accumulate into out when accumulate != 0).  Used for the reductions of
 * per-tile partial gradients.
 */
sparc_status sparc_column_sum(int64_t rows, int64_t cols, const float* in,
                              float* out, int accumulate, sparc_stream_t stream);

const char* sparc_last_error(void);
const char* sparc_version(void);

/* ---------------------------------------------------------------------------
 * The module's sequence path, fused (SPARCMixer forward and backward): the
 * P1 controls, the gain*tanh write, the scan and the relu(cat) epilogue
 * read x directly, with no [B,T,M] write tensors.
 *
 * x [B,T,2M] (io_dtype; x[..., :M] feeds the real parts, x[..., M:] the
 * imaginary ones), directions [2M+1] fp32 (the last entry is the bias),
 * parameters [M] fp32.  M must be a multiple of 4; x, y, dy, dx and the
 * directions 16-byte aligned.  With length 0 the per-token tensors (x, y,
 * h_re, h_im, eta, delta, dy, dx, deta, ddelta) are neither read nor written
 * and may be NULL; the last state is zero and every gradient is zero.
 * ------------------------------------------------------------------------- */
/* Workspace bytes of sparc_mixer_forward (direction 0) or _backward (1); 0 if
 * the shape is invalid. */
size_t sparc_mixer_workspace_bytes(int64_t batch, int64_t length, int64_t modes, int direction);

/* eta, delta [B*T] fp32: the controls eta = log16 tanh(x.u_r + b_r), delta =
 * (pi/2) tanh(x.u_p + b_p).  y [B,T,2M] = relu(cat(h_re, h_im)) and h_re,
 * h_im [B,T,M] (the states, kept for the backward) in io_dtype.  last_re,
 * last_im [B,M] fp32: the state after step T-1 (both NULL: not written).
 * Replaces run_sequence's P1 path: make_controls and make_scan_inputs
 * (sparc-kernal/forward/control.py:129-195), _SPARCChunkScan.forward
 * (sparc-kernal/backward/scan.py:1126-1372) and the output epilogue
 * (sparc-kernal/forward/scan.py:1598-1603). */
sparc_status sparc_mixer_forward(int64_t batch, int64_t length, int64_t modes, int32_t io_dtype,
                                 const void* x, const float* phase_direction, const float* radial_direction,
                                 const float* nu_log, const float* theta_log, const float* write_log_gain,
                                 const float* write_phase_response, const float* write_radial_response,
                                 float* eta, float* delta, void* y, void* h_re, void* h_im,
                                 float* last_re, float* last_im, void* workspace, size_t workspace_bytes,
                                 sparc_stream_t stream);

/* The forward's scan alone, with the controls given: eta, delta [B*T] fp32
 * are inputs (a caller that has them more cheaply, e.g. folded into the
 * projection that produces x, skips the two dot products over x).  Outputs
 * as sparc_mixer_forward.  Replaces _SPARCChunkScan.forward with the write
 * and epilogue fused (sparc-kernal/backward/scan.py:1126-1372,
 * forward/control.py:141-195, forward/scan.py:1598-1603). */
sparc_status sparc_mixer_scan_forward(int64_t batch, int64_t length, int64_t modes, int32_t io_dtype,
                                      const void* x, const float* eta, const float* delta, const float* nu_log,
                                      const float* theta_log, const float* write_log_gain,
                                      const float* write_phase_response, const float* write_radial_response,
                                      void* y, void* h_re, void* h_im, float* last_re, float* last_im,
                                      void* workspace, size_t workspace_bytes, sparc_stream_t stream);

/* The backward of sparc_mixer_scan_forward: dx [B,T,2M] (io_dtype) through
 * the write only, deta, ddelta [B*T] fp32 (the gradients of the controls)
 * and the five parameter gradients [M] fp32 (overwritten); the controls'
 * own backward is the caller's.  Workspace: sparc_mixer_workspace_bytes(...,
 * 1).  Replaces _SPARCChunkScan.backward (sparc-kernal/backward/scan.py:
 * 1375-1640) and _LatestSPARCWrite.backward (backward/control.py:92-129). */
sparc_status sparc_mixer_scan_backward(int64_t batch, int64_t length, int64_t modes, int32_t io_dtype,
                                       const void* x, const float* eta, const float* delta, const float* nu_log,
                                       const float* theta_log, const float* write_log_gain,
                                       const float* write_phase_response, const float* write_radial_response,
                                       const void* h_re, const void* h_im, const void* dy, const float* dlast_re,
                                       const float* dlast_im, void* dx, float* deta, float* ddelta, float* dnu_log,
                                       float* dtheta_log, float* dwrite_log_gain, float* dwrite_phase_response,
                                       float* dwrite_radial_response, void* workspace, size_t workspace_bytes,
                                       sparc_stream_t stream);

/* dy [B,T,2M] (io_dtype): the gradient of y; dlast_re, dlast_im [B,M] fp32:
 * of the last state (both NULL: zero).  eta, delta, h_re, h_im as the
 * forward wrote them.  Writes dx [B,T,2M] (io_dtype) and, overwriting, the
 * direction gradients [2M+1] and the parameter gradients [M] (fp32).
 * Deterministic (fixed-order reductions).
 *
 * Forms (sparc_mixer_backward_form): where no time segments are needed (at
 * least 1024 chains of 64 modes), T > 0 and every chain fits on the GPU at
 * once at the kernel's occupancy, the call runs in ONE launch that also
 * completes dx and the direction gradients: the chains of a batch row
 * exchange per-block sums through the workspace (no atomics: each block has
 * one owner chain, which sums the row's records in a fixed order once all
 * are stored) and each chain completes a block eight blocks (fp32: four)
 * after computing it.  Its waits are bounded (sparc_set_wait_limit): a wait
 * that reaches the bound sets the workspace error word
 * (sparc_scan_workspace_error) and leaves NaN gradients for that block, and
 * every workgroup still finishes.  Otherwise the time pieces below, else one
 * scan launch followed by the controls' backward.
 *
 * Streams: when T splits into time pieces (T a multiple of 256, and at least
 * 1024 chains of 64 modes, so that no time segments are needed; the
 * workspace query covers both layouts), the call runs the
 * pieces last first and launches each piece's controls backward on a second
 * stream, so that it overlaps the next piece's scan.  That stream is owned by
 * the library: one per device, non-blocking, default priority, created with
 * its events on the first such call that is not under graph capture and kept
 * until the process ends.  Every use of it is bracketed by events: it first
 * waits for the given stream, and the given stream waits for it before the
 * call's last reductions and before any error return after that fork, so
 * work enqueued afterwards on the given stream sees every result.  If the
 * stream or an event call is unavailable (the first call is under capture, a
 * HIP call fails), the same launches go to the given stream alone, with the
 * same results.  Under capture the fork and join become graph edges and
 * nothing waits on the host.  A process-wide mutex is held while a call
 * enqueues, so calls from several host threads do not share an event between
 * a record and its wait.
 *
 * Replaces _SPARCChunkScan.backward (sparc-kernal/backward/scan.py:1375-1640),
 * _LatestSPARCWrite.backward (sparc-kernal/backward/control.py:92-129, kernel
 * :10-89) and the autograd of make_controls' F.linear
 * (sparc-kernal/forward/control.py:129-139). */
sparc_status sparc_mixer_backward(int64_t batch, int64_t length, int64_t modes, int32_t io_dtype,
                                  const void* x, const float* phase_direction, const float* radial_direction,
                                  const float* nu_log, const float* theta_log, const float* write_log_gain,
                                  const float* write_phase_response, const float* write_radial_response,
                                  const float* eta, const float* delta, const void* h_re, const void* h_im,
                                  const void* dy, const float* dlast_re, const float* dlast_im, void* dx,
                                  float* dphase_direction, float* dradial_direction, float* dnu_log,
                                  float* dtheta_log, float* dwrite_log_gain, float* dwrite_phase_response,
                                  float* dwrite_radial_response, void* workspace, size_t workspace_bytes,
                                  sparc_stream_t stream);

/* The form sparc_mixer_backward takes for this shape on the current device:
 * 2 (one launch), 1 (time pieces), 0 (one scan launch, then the controls'
 * backward), -1 (invalid shape).  No counterpart in the reference (one Triton
 * launch sequence). */
int sparc_mixer_backward_form(int64_t batch, int64_t length, int64_t modes, int32_t io_dtype);

/* Process-wide: 0 (default) lets sparc_mixer_backward take the one-launch
 * form wherever it applies, 1 never.  Returns the previous setting (-1 for
 * an invalid argument).  For tests and A/B measurements, and for callers
 * that keep other kernels running on the same GPU beside the backward (the
 * one-launch form's waits last until all of its chains are resident); no
 * counterpart in the reference. */
int sparc_mixer_backward_plan(int plan);

/* ---- the controls alone (make_controls) ----------------------------------
 * Rows x [rows, width] (io_dtype, width a positive multiple of 8, 16-byte
 * aligned) against two directions [width + 1] fp32 (the bias last, 16-byte
 * aligned): delta = pi/2 tanh(x.phase_direction), eta = log16
 * tanh(x.radial_direction), one fp32 value per row.  The mixer entry points
 * above run the same kernels over the module's input (width 2M); these take
 * any width, e.g. a normalised input whose projection the directions have
 * been folded into.  With rows = 0 nothing is read or written (the
 * pointers may be NULL).  Replaces make_controls
 * (sparc-kernal/forward/control.py:129-139). */
sparc_status sparc_controls_forward(int64_t rows, int64_t width, int32_t io_dtype, const void* x,
                                    const float* phase_direction, const float* radial_direction, float* eta,
                                    float* delta, sparc_stream_t stream);

/* Workspace bytes of sparc_controls_backward (0: invalid shape). */
size_t sparc_controls_workspace_bytes(int64_t rows, int64_t width);

/* The backward of sparc_controls_forward given deta, ddelta [rows] fp32:
 * dx [rows, width] (io_dtype) += dp_phase * phase_direction + dp_radial *
 * radial_direction in place (dp: the gradients of the two dot products), and
 * the direction gradients [width + 1] fp32, bias last, overwritten (zero
 * with rows = 0; the row tensors and the workspace may then be NULL).
 * Deterministic.  Replaces the autograd of make_controls' tanh and F.linear
 * (sparc-kernal/forward/control.py:129-139). */
sparc_status sparc_controls_backward(int64_t rows, int64_t width, int32_t io_dtype, const void* x,
                                     const float* phase_direction, const float* radial_direction, const float* eta,
                                     const float* delta, const float* deta, const float* ddelta, void* dx,
                                     float* dphase_direction, float* dradial_direction, void* workspace,
                                     size_t workspace_bytes, sparc_stream_t stream);

/* ---- the controls folded into an input projection ------------------------
 * weight [width, dim] (io_dtype, 16-byte aligned, dim a positive multiple of
 * 8 up to 4096) is the projection W with x = x_n W^T; the directions [width
 * + 1] fp32 (bias last).  sparc_controls_fold writes the folded directions
 * [dim + 1] fp32: folded[d] = sum_w direction[w] W[w, d], folded[dim] =
 * direction[width], the sums in a fixed order, so that sparc_controls_forward
 * over x_n with them gives the controls of x.  sparc_controls_fold_backward
 * maps the gradients of the folded directions [dim + 1] back:
 * ddirection[w] = sum_d dfolded[d] W[w, d], ddirection[width] =
 * dfolded[dim]; with dweight (io_dtype [width, dim], 16-byte aligned; NULL:
 * skipped) it also adds the folded directions' share of the projection's
 * gradient in place, dweight[w, d] += phase[w] dfolded_phase[d] +
 * radial[w] dfolded_radial[d] (fp32, rounded once); the directions may be
 * NULL without dweight.  No counterpart in the reference, which ships the
 * layer, not a network: the 12-layer stack that runs the layer in its
 * training configuration folds its controls this way. */
size_t sparc_controls_fold_workspace_bytes(int64_t width, int64_t dim);
sparc_status sparc_controls_fold(int64_t width, int64_t dim, int32_t io_dtype, const void* weight,
                                 const float* phase_direction, const float* radial_direction, float* folded_phase,
                                 float* folded_radial, void* workspace, size_t workspace_bytes,
                                 sparc_stream_t stream);
sparc_status sparc_controls_fold_backward(int64_t width, int64_t dim, int32_t io_dtype, const void* weight,
                                          const float* phase_direction, const float* radial_direction,
                                          const float* dfolded_phase, const float* dfolded_radial,
                                          float* dphase_direction, float* dradial_direction, void* dweight,
                                          sparc_stream_t stream);

/* ---- RMSNorm (the block stack's pre-norm and final norm) -----------------
 * x, y [rows, cols] and weight [cols] in io_dtype (cols a positive multiple
 * of 8 up to 4096; x, y and weight 16-byte aligned); rstd [rows] fp32.
 * Forward: rstd = 1 / sqrt(mean over the row of x^2 + eps), y = (x rstd)
 * weight, in fp32 arithmetic.  No counterpart in the reference, which ships
 * the layer, not a network: torch.nn.RMSNorm's formula for the 12-layer
 * stack that runs the layer in its training configuration. */
sparc_status sparc_rms_norm_forward(int64_t rows, int64_t cols, int32_t io_dtype, const void* x, const void* weight,
                                    float eps, void* y, float* rstd, sparc_stream_t stream);

/* Workspace bytes of sparc_rms_norm_backward (0: invalid shape). */
size_t sparc_rms_norm_workspace_bytes(int64_t rows, int64_t cols);

/* Backward of sparc_rms_norm_forward given rstd from it and dy [rows, cols]
 * (io_dtype): dx = rstd (g - xhat mean(g xhat)) with xhat = x rstd, g = dy
 * weight (io_dtype, 16-byte aligned), and dweight [cols] fp32 = the sum over
 * rows of dy xhat, overwritten, in a fixed order (zero with rows = 0; the row
 * tensors and the workspace may then be NULL). */
sparc_status sparc_rms_norm_backward(int64_t rows, int64_t cols, int32_t io_dtype, const void* x, const void* weight,
                                     const float* rstd, const void* dy, void* dx, float* dweight, void* workspace,
                                     size_t workspace_bytes, sparc_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* SPARC_HIP_H */
