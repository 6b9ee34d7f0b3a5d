/*
 * fields_amd.h — C ABI of the MI355X (gfx950) Field-block hot path.
 *
 * The Field recurrence of Fields LM, per (batch b, time t, channel c), C = d_model / 2:
 *
 *   inj   = tanh(raw[b,t,c]) + i*tanh(raw[b,t,C+c])
 *   v     = 0.9 * sigmoid(raw[b,t,2C+c])              (independent vacancy)
 *   lam   = tr[c] + i*ti[c]
 *   disp  = v * lam * s[t-1]                          (displaced readout)
 *   s[t]  = (1 - v) * lam * s[t-1] + gamma[c]*v*inj   (causal write), s[-1] = state_in or 0
 *   read[b,t,:] = [Re s | Im s | Re disp | Im disp]   (4C floats)
 *
 * All pointers are device pointers unless stated. Every entry point is stream-ordered on
 * `stream`, performs no allocation and no host synchronisation (so a caller may capture it
 * in a hipGraph), keeps no global mutable state and is reentrant: calls on different
 * streams must use different workspaces. The one exception is fl_scan_forward_static, whose
 * look-back state is a per-GPU array inside the library (see its comment).
 *
 * Complex state vectors are stored planar, [B, 2C] floats: the first C entries of a row
 * are the real parts and the next C the imaginary parts (the layout of read[:, t, :2C]).
 *
 * Return value: FL_OK or one of the FL_ERR_* codes below. FL_ERR_HIP_BASE + e means that
 * HIP reported error e (a hipError_t) on launch.
 */
#ifndef FIELDS_AMD_H_
#define FIELDS_AMD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element types of raw / read buffers */
#define FL_DTYPE_F32 0
#define FL_DTYPE_BF16 1

/* algorithm selector for fl_scan_forward_ex (low 8 bits); bits 8.. select a tiling variant of
 * FL_ALGO_LOOKBACK for tuning: 0 = default (LDS-staged 16-byte loads and stores where raw is bf16
 * with 16-byte aligned rows, read is fp32 and C is a multiple of 64; register loads and stores
 * otherwise), 1..5 = other tilings, 6 = LDS-staged where possible, 7 = default tiling with
 * register loads and stores on every input */
#define FL_ALGO_AUTO 0
#define FL_ALGO_CHUNKED3 1 /* chunk summary -> chunk carry -> chunk materialise (three launches) */
#define FL_ALGO_LOOKBACK 2 /* single launch, decoupled look-back across chunks (default) */

#define FL_OK 0
#define FL_ERR_INVALID_ARGUMENT 1 /* shape / stride / pointer check failed (Python: ValueError) */
#define FL_ERR_DTYPE 2            /* unsupported raw or read dtype (Python: TypeError) */
#define FL_ERR_WORKSPACE 3        /* workspace NULL or smaller than fl_scan_workspace_bytes */
#define FL_ERR_CAPTURE 4          /* fl_scan_forward_static: first call on a device under capture */
#define FL_ERR_HIP_BASE 1000      /* FL_ERR_HIP_BASE + hipError_t */

/*
 * Chunked forward scan over a whole sequence batch.
 *
 * Replaces `fused_field_read(raw, transition_r, transition_i, gamma, block_c, chunk_t)`
 * (src/fields_official/reference/field_only_v4_chunked_triton_wiki100.py:1108-1123) and the
 * three Triton launches of `_ChunkedFieldReadFunction.forward` (same file, 913-1018:
 * `_field_chunk_summary_kernel` 443-516, `_field_chunk_carry_kernel` 519-550,
 * `_field_chunk_materialize_kernel` 553-622). The reference always starts from state 0 and
 * takes fp32 raw only; state_in/state_out and bf16 raw are extensions (state_in = NULL and
 * fp32 raw reproduce the reference call).
 *
 *   raw        [B, T, 3C] of raw_dtype; element (b,t,j) at raw + b*raw_stride_b + t*raw_stride_t + j
 *              (strides in elements, channel stride 1, raw_stride_t >= 3C)
 *   tr, ti, gamma  [C] fp32
 *   state_in   [B, 2C] fp32 planar, or NULL for the zero state
 *   state_out  [B, 2C] fp32 planar, or NULL; receives s[T-1]
 *   read       [B, T, 4C] contiguous, read_dtype: FL_DTYPE_F32, or FL_DTYPE_BF16 (values rounded
 *              to nearest even; 7,168 instead of 11,264 bytes per token at C = 512 with bf16 raw)
 *   workspace  device scratch of at least fl_scan_workspace_bytes(B, T, C) bytes, 256-byte
 *              aligned, ZERO-FILLED before its first use and then reused as is: its first 2 KiB
 *              hold launch counters that every call leaves ready for the next one. Calls on one
 *              workspace must be stream-ordered (one workspace per stream). Every launch advances
 *              an epoch kept there; the launch at each 2^30-launch wrap of its tag bits zero-fills
 *              the rest of the workspace itself, so it is never zero-filled again by the caller.
 *   workspace_bytes  the size of that allocation. It must not exceed the allocation: the wrap
 *              launch zero-fills workspace_bytes after the header (every word an earlier call at
 *              any shape may have left), so a larger value writes past the buffer.
 *
 * Workspace header (first 2 KiB; little-endian words at these byte offsets):
 *   128  u32  error word: bit 0 a bounded wait gave up, bit 1 a ticket beyond the launch's tiles
 *             (set by the kernels, never cleared by them)
 *   384  u32  spin limit: polls before a wait gives up (0 = 2^20); written by the caller
 *   392  u64  address of a host-visible (pinned, device-mapped) u32 that the kernels set non-zero
 *             whenever they set the error word, so a caller can see a failure without reading
 *             device memory; 0 = none; written by the caller
 * A wait that gives up makes what depends on it NaN (the tile's outputs and every later tile of
 * its chain, a row's RMSNorm scale, the backward's gradients), so an output computed without a
 * value it needed cannot pass for a valid one. The same header leads the backward's workspace.
 */
int fl_scan_forward(const void* raw, int raw_dtype, int64_t B, int64_t T, int64_t C,
                    int64_t raw_stride_b, int64_t raw_stride_t, const float* tr, const float* ti,
                    const float* gamma, const float* state_in, float* state_out, void* read,
                    int read_dtype, void* workspace, size_t workspace_bytes, void* stream);

/*
 * fl_scan_forward without a workspace argument, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). It has no
 * counterpart in the reference. It calls no hipMalloc, hipFree or allocating library routine: the
 * look-back state lives in a file-scope device array of FL_STATIC_SCRATCH_BYTES in this library,
 * one copy per GPU, held until the process ends.
 *
 *   * Shapes: B * ceil(C / 64) * ceil(T / 128) <= FL_STATIC_MAX_TILES (config 2 needs 1,024,
 *     B = 1 with T = 65,536 and C = 512 needs 4,096); larger shapes return FL_ERR_WORKSPACE.
 *   * The first call on each device zero-fills that device's array on `stream`: it must not be
 *     made under stream capture (FL_ERR_CAPTURE). Later calls may be captured.
 *   * Every call on one GPU shares that GPU's array: calls that overlap on one GPU (two streams,
 *     two threads) race and must be serialised by the caller.
 *   * A bounded wait that gives up leaves NaN in the outputs that depend on it (there is no error
 *     word the caller can read).
 * Arguments and results as fl_scan_forward (FL_ALGO_AUTO); results are bit-identical to it.
 */
#define FL_STATIC_MAX_TILES 12288
#define FL_STATIC_SCRATCH_BYTES 31508480 /* 2 KiB header + 12,288 status words + tagged words */
int fl_scan_forward_static(const void* raw, int raw_dtype, int64_t B, int64_t T, int64_t C,
                           int64_t raw_stride_b, int64_t raw_stride_t, const float* tr,
                           const float* ti, const float* gamma, const float* state_in,
                           float* state_out, void* read, int read_dtype, void* stream);

/* As fl_scan_forward with an explicit algorithm (FL_ALGO_*). */
int fl_scan_forward_ex(const void* raw, int raw_dtype, int64_t B, int64_t T, int64_t C,
                       int64_t raw_stride_b, int64_t raw_stride_t, const float* tr,
                       const float* ti, const float* gamma, const float* state_in,
                       float* state_out, void* read, int read_dtype, void* workspace,
                       size_t workspace_bytes, int algo, void* stream);

/*
 * Forward scan with the mixer's read_norm RMSNorm fused into the epilogue: writes
 *
 *   out[b,t,j] = (read[b,t,j] * rsqrt(sum_i read[b,t,i]^2 / (4C) + eps)) * norm_weight[j]
 *
 * for the read that fl_scan_forward computes (in fp32), without writing read itself. Replaces
 * `self.read_norm(fused_field_read(...))` in `IndependentVacancyField.forward`
 * (field_only_v4_chunked_triton_wiki100.py:1176-1193, RMSNorm 300-309); the out_proj GEMM
 * then reads `out` directly. out_dtype FL_DTYPE_BF16 gives the fp32 value rounded to nearest
 * even, which is what the reference's out_proj sees under bf16 autocast.
 *
 * Arguments as fl_scan_forward, plus norm_weight [4C] fp32 and eps (>= 0); the same workspace.
 * Single-launch path only; C <= 4096.
 */
int fl_scan_norm_forward(const void* raw, int raw_dtype, int64_t B, int64_t T, int64_t C,
                         int64_t raw_stride_b, int64_t raw_stride_t, const float* tr,
                         const float* ti, const float* gamma, const float* state_in,
                         float* state_out, const float* norm_weight, float eps, void* out,
                         int out_dtype, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Backward of fl_scan_forward: the gradients of a loss L given dL/dread (and dL/dstate_out).
 *
 * Replaces `_ChunkedFieldReadFunction.backward`
 * (field_only_v4_chunked_triton_wiki100.py:1020-1105; Triton kernels 625-910: chunk summary,
 * chunk carry, chunk materialise, then a torch sum of the parameter partials). Two launches on
 * `stream`: the reverse scan (decoupled look-back over chunks taken in reverse time order), whose
 * tiles write per-tile parameter-gradient partials into the workspace, then a reduction that adds
 * them up in a fixed order (bit-reproducible).
 *
 *   raw, strides, tr, ti, gamma, state_in   as given to the forward call
 *   read            [B, T, 4C] fp32, the forward output (the state planes at every 8th row
 *                   are read: the state before each 8-step group, from which s_{t-1} of the
 *                   group's steps is recomputed; the reference reads it back at every step)
 *   grad_read       [B, T, 4C] fp32 contiguous
 *   grad_state_out  [B, 2C] fp32 planar, or NULL (state_out unused)
 *   grad_raw        [B, T, 3C] contiguous, grad_raw_dtype F32 or BF16 (overwritten)
 *   grad_tr, grad_ti, grad_gamma  [C] fp32 (overwritten)
 *   grad_state_in   [B, 2C] fp32 planar, or NULL
 *   workspace       >= fl_scan_backward_workspace_bytes(B, T, C), 256-byte aligned, zero-filled
 *                   before first use, then reused (one per stream), as for fl_scan_forward;
 *                   workspace_bytes must not exceed the allocation (the same wrap clear)
 * A block that finds the ticket counter out of range (error bit 1) computes nothing, so the
 * parameter gradients of that call are NaN (its reduction sums every tile's partials).
 */
int fl_scan_backward(const void* raw, int raw_dtype, int64_t B, int64_t T, int64_t C,
                     int64_t raw_stride_b, int64_t raw_stride_t, const float* tr, const float* ti,
                     const float* gamma, const float* state_in, const float* read,
                     const float* grad_read, const float* grad_state_out, void* grad_raw,
                     int grad_raw_dtype, float* grad_tr, float* grad_ti, float* grad_gamma,
                     float* grad_state_in, void* workspace, size_t workspace_bytes, void* stream);

/* Workspace size in bytes for fl_scan_backward (host function, no device call). Replaces the
 * ten [B, n_chunks, C] torch.empty buffers of field_only_v4_chunked_triton_wiki100.py:1027-1037. */
size_t fl_scan_backward_workspace_bytes(int64_t B, int64_t T, int64_t C);

/*
 * Workspace size in bytes for fl_scan_forward at this shape (host function, no device call).
 * Replaces the six [B, n_chunks, C] fp32 torch.empty buffers of
 * field_only_v4_chunked_triton_wiki100.py:941-952.
 */
size_t fl_scan_workspace_bytes(int64_t B, int64_t T, int64_t C);

/*
 * Single-token recurrent step for the decode loop: reads state (s[t-1]) and raw_t, writes
 * read_t and overwrites state with s[t], in one pass.
 *
 * The reference has no incremental step; this is the per-t body of
 * `_field_chunk_materialize_kernel` (field_only_v4_chunked_triton_wiki100.py:583-621) applied
 * to one token with the state carried between calls. Equal to row t of fl_scan_forward.
 *
 *   raw_t  [B, 3C] of raw_dtype, row stride raw_stride_b elements (>= 3C), channel stride 1
 *   state  [B, 2C] fp32 planar, updated in place
 *   read_t [B, 4C] contiguous, read_dtype FL_DTYPE_F32
 */
int fl_decode_step(const void* raw_t, int raw_dtype, int64_t B, int64_t C, int64_t raw_stride_b,
                   const float* tr, const float* ti, const float* gamma, float* state,
                   void* read_t, int read_dtype, void* stream);

/*
 * fl_decode_step with the read_norm RMSNorm fused in: state advances as in fl_decode_step and
 * out_t [B, 4C] (out_dtype F32 or BF16, contiguous) receives the normalised read_t, as
 * fl_scan_norm_forward defines it. The decode-loop counterpart of fl_scan_norm_forward
 * (field_only_v4_chunked_triton_wiki100.py:1176-1193 and 300-309 for one token).
 */
int fl_decode_norm_step(const void* raw_t, int raw_dtype, int64_t B, int64_t C,
                        int64_t raw_stride_b, const float* tr, const float* ti,
                        const float* gamma, float* state, const float* norm_weight, float eps,
                        void* out_t, int out_dtype, void* stream);

/*
 * Boundary scan of the softpatch mixer: s[b,t,r] = a[b,t] * s[b,t-1,r] + drive[b,t,r] with
 * s[b,-1,:] = state_in (or 0), written to out [B, T, R]; state_out [B, R] receives s[b,T-1,:].
 *
 * Replaces `hierarchical_scan(a, drive, block=32)` in `BoundaryStateMixer.forward`
 * (src/fields_official/reference/official_source/field_hybrid_attentionfree_qualification_v3.py:458-460
 * and field_hybrid_speed_optimization_v6.py:333-335), where a = 1 - boundary is one value per
 * token broadcast over the rank R. All buffers fp32 and contiguous; state_in / state_out may be
 * NULL. No workspace.
 */
int fl_boundary_scan(const float* a, const float* drive, int64_t B, int64_t T, int64_t R,
                     const float* state_in, float* state_out, float* out, void* stream);

/*
 * Field block elementwise tail for inference, one launch per row block:
 *   x_new  = x + out * sigmoid(gate_pre)            (IndependentVacancyField.forward return,
 *                                                    field_only_v4_chunked_triton_wiki100.py:1193-1195)
 *   normed = RMSNorm(x_new) * norm_weight           (FieldBlock.ff_norm, same file 1219-1221, 300-309)
 * out / gate_pre are the out_proj / gate_proj GEMM outputs (g_dtype), x / x_new / normed the
 * residual stream (x_dtype); all [rows, dim] contiguous except gate_pre, whose rows lie
 * gate_stride >= dim elements apart (a column slice of a GEMM output that also holds other
 * columns, e.g. write_proj and gate_proj computed in one GEMM). Every intermediate is rounded where
 * the stock ops round it (bf16 ops compute in fp32 and round their result).
 */
int fl_gate_residual_norm(const void* x, int x_dtype, const void* out, const void* gate_pre,
                          int g_dtype, int64_t rows, int64_t dim, int64_t gate_stride,
                          const float* norm_weight, float eps, void* x_new, void* normed,
                          void* stream);

/*
 * SwiGLU activation of the Field block FFN (PackedSwiGLU.forward, same file 312-325):
 * out[r, j] = silu(gate_up[r, j]) * gate_up[r, hidden + j], [rows, 2*hidden] -> [rows, hidden].
 */
int fl_swiglu(const void* gate_up, int dtype, int64_t rows, int64_t hidden, void* out,
              void* stream);

/* Library version string (host function). No counterpart in the reference. */
const char* fl_version(void);

#ifdef __cplusplus
}
#endif

#endif /* FIELDS_AMD_H_ */
