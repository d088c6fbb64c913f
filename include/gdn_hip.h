/*
 * gdn_hip.h -- C ABI of libgdn_hip.so, the MI355X (gfx950) kernels of the
 * Gated DeltaNet linear-attention path.
 *
 * Every entry point takes device pointers wrapped in plain tensor descriptors
 * (pointer, dtype, shape, element strides; gdn_hbm_copy, a measurement
 * utility, takes plain pointers), launches on the caller's HIP
 * stream, never allocates, never synchronises the host and keeps no global
 * mutable state (one exception: paged_attention_decode_noalloc works in a
 * static device array shared by its calls on a GPU and caches that array's
 * address per device).  Return value: 0 on success, > 0 a hipError_t from the
 * launch, < 0 a validation code (nothing was launched).  gdn_strerror() maps
 * any code to text.
 *
 * Index semantics shared by all entry points:
 *  - state / conv-state slot indices are int32 or int64; a slot outside
 *    [0, num_slots) marks a padding sequence: its output rows are zero and no
 *    state is read or written.  Slots of one call must be distinct.
 *  - cu_seqlens is int32 or int64, length N+1, non-decreasing, cu[0] = 0,
 *    cu[N] <= T.  Kernels clamp every sequence range to [0, T].
 *
 * Reference interface (paths relative to yuyifanbupt/myvllm src/myvllm):
 *  - gdn_recurrent_step   <- recurrent_gated_delta_rule,
 *                            ops/gated_delta_rule/gated_delta_rule.py:69-92
 *                            (kernel ops/gated_delta_rule/fused_recurrent_gdn.py:105-166)
 *  - gdn_chunk_prefill    <- chunk_gated_delta_rule,
 *                            ops/gated_delta_rule/gated_delta_rule.py:31-66
 *  - causal_conv1d_varlen <- causal_conv1d_fn, ops/causal_conv1d.py:221-273
 *  - causal_conv1d_step   <- causal_conv1d_update, ops/causal_conv1d.py:434-470
 *  - gdn_rms_norm_gated   <- RMSNormGated, layers/norm.py:44-58
 *  - gdn_gating           <- the gates of GatedDeltaNet.forward,
 *                            layers/linear_attention.py:89-90
 *  - causal_conv1d_varlen_qknorm <- causal_conv1d_fn + the L2 norm of
 *                            layers/linear_attention.py:113-114, one launch
 *  - gdn_decode_step_fused <- the decode branch of GatedDeltaNet.forward,
 *                            layers/linear_attention.py:89-90 (gating), :95
 *                            (causal_conv1d_update), :113-114 (L2 norm), :119
 *                            (recurrent_gated_delta_rule), one launch instead of four
 *  - flash_attention_varlen  <- flash_attention_prefill, ops/full_attention.py:114-173
 *  - paged_attention_prefill <- paged_flash_attention_prefill, ops/full_attention.py:454-512
 *  - paged_attention_decode  <- paged_flash_attention_decode, ops/full_attention.py:282-335
 */
#ifndef GDN_HIP_H_
#define GDN_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GDN_ABI_VERSION 1

/* element types */
#define GDN_DTYPE_F32 0
#define GDN_DTYPE_BF16 1
#define GDN_DTYPE_F16 2
#define GDN_DTYPE_I32 3
#define GDN_DTYPE_I64 4

/* validation codes (negative); positive codes are hipError_t values */
#define GDN_OK 0
#define GDN_ERR_NULL (-1)       /* missing descriptor or data pointer */
#define GDN_ERR_NDIM (-2)       /* wrong number of dimensions */
#define GDN_ERR_SHAPE (-3)      /* shapes disagree with each other */
#define GDN_ERR_DTYPE (-4)      /* unsupported element type */
#define GDN_ERR_STRIDE (-5)     /* innermost stride must be 1 (state: [K][V] contiguous) */
#define GDN_ERR_HEADS (-6)      /* num_v_heads not a positive multiple of num_k_heads */
#define GDN_ERR_HEAD_DIM (-7)   /* head dims not supported by the kernels */
#define GDN_ERR_CHUNK (-8)      /* chunk size not supported */
#define GDN_ERR_ALIGN (-9)      /* pointer/stride misaligned for 16-byte vector access */
#define GDN_ERR_CONV_WIDTH (-10) /* conv width outside [2, 6] */
#define GDN_ERR_RANGE (-11)     /* a size exceeds the kernels' index range */
#define GDN_ERR_SCRATCH (-12)   /* the call needs more than the library's static scratch holds */
#define GDN_ERR_ARG (-13)       /* an option argument is out of range */

#define GDN_MAX_NDIM 4

typedef struct gdn_tensor {
  void* data;                    /* device pointer (may be NULL only if numel == 0) */
  int32_t dtype;                 /* GDN_DTYPE_* */
  int32_t ndim;                  /* 1..4 */
  int64_t shape[GDN_MAX_NDIM];   /* sizes */
  int64_t stride[GDN_MAX_NDIM];  /* strides in elements */
} gdn_tensor;

/*
 * Fused recurrent decode step, one token per sequence (replaces
 * recurrent_gated_delta_rule, ops/gated_delta_rule/gated_delta_rule.py:69-92).
 *   q, k   : (B, Hk, K)  bf16|f16|f32, last stride 1
 *   v      : (B, Hv, V)  same dtype as q
 *   g      : (B, Hv)     f32|bf16|f16   natural-log decay
 *   beta   : (B, Hv)     f32|bf16|f16
 *   state  : (S, Hv, K, V) f32, [K][V] contiguous per head; updated in place
 *   state_indices : (B,) i32|i64
 *   out    : (B, Hv, V)  bf16|f16|f32, last stride 1
 * Per (b, h): S <- e^g S; d = beta (v - S^T k); S += k d^T; o = S^T (scale q).
 * Head dims: K and V multiples of 8 up to 256 (64 x 64, 128 x 128 and
 * 256 x 256 have their own kernels; other shapes run zero-padded in the
 * 128 x 128 one, or the 256 x 256 one when either dim exceeds 128).
 */
int gdn_recurrent_step(const gdn_tensor* q, const gdn_tensor* k, const gdn_tensor* v,
                       const gdn_tensor* g, const gdn_tensor* beta, gdn_tensor* state,
                       const gdn_tensor* state_indices, gdn_tensor* out, float scale,
                       void* stream);

/*
 * Chunked gated-delta-rule prefill over packed varlen sequences (replaces
 * chunk_gated_delta_rule, ops/gated_delta_rule/gated_delta_rule.py:31-66).
 *   q, k   : (T, Hk, K)  bf16|f16, last stride 1, token/head strides multiples of 8
 *   v      : (T, Hv, V)  same dtype as q, same constraints
 *   g      : (T, Hv)     f32   natural-log decay per token and v-head
 *   beta   : (T, Hv)     f32|bf16|f16
 *   state  : (S, Hv, K, V) f32; initial state read from state[idx[n]], final
 *            state written back there
 *   state_indices : (N,) i32|i64
 *   cu_seqlens    : (N+1,) i32|i64
 *   out    : (T, Hv, V)  v's dtype, last stride 1
 * chunk_size must be 64; K and V multiples of 8 from 8 to 128 (the
 * reference's k_head_dim <= 128, ops/gated_delta_rule/h.py:211; head dims
 * below 128 run zero-padded to 128, at the cost of 128).  Output rows of
 * tokens no sequence covers ([0, cu[0]) and [cu[N], T)) are set to zero, as
 * the reference allocates o zero-filled (ops/gated_delta_rule/o.py:147).
 * Range: the MFMA operands are fp16, so every q and k row must have an L2
 * norm of at most 128 (the layer's rows are L2-normalised, norm 1) and |v|
 * entries must stay below 65504 (an fp16 out also overflows past 65504, as
 * the reference's fp16 output would); the state may have any magnitude (it is
 * held in per-column power-of-two units).  Keys of any norm in that range
 * keep the fp32 state bound (the state-update split is sized from each
 * chunk's largest key norm).
 * Failure: the kernel's wave roles hand work to each other through bounded
 * waits; a wait that gives up (a pipeline error, never expected) writes NaN
 * to all output rows of that (sequence, v-head) and leaves its state slot
 * untouched.  The environment plays no part in a call.
 */
int gdn_chunk_prefill(const gdn_tensor* q, const gdn_tensor* k, const gdn_tensor* v,
                      const gdn_tensor* g, const gdn_tensor* beta, gdn_tensor* state,
                      const gdn_tensor* state_indices, const gdn_tensor* cu_seqlens,
                      gdn_tensor* out, float scale, int32_t chunk_size, void* stream);

/*
 * gdn_chunk_prefill with options (no counterpart in the reference).  With
 * flags = 0, items_per_wg = -1 and spin_limit = -1 it is gdn_chunk_prefill.
 *   flags: GDN_PREFILL_ZERO_INIT    every sequence starts from a zero state
 *                                   (its slot is not read);
 *          GDN_PREFILL_ACCUM_STATE  the final state is added to the slot
 *                                   instead of replacing it;
 *          GDN_PREFILL_ACCUM_OUT    o is added to out (fp32 out only); rows of
 *                                   padding or uncovered tokens are left as they are.
 *   out may be fp32 when q, k and v are fp16 (v's dtype otherwise).  These
 *   serve fp32 q/k/v: the recurrence is linear in (state, v), so with
 *   v = v_hi + v_lo (fp16 each) one call with v_hi and fp32 out and a second
 *   with v_lo, ZERO_INIT | ACCUM_STATE | ACCUM_OUT give the result for v.
 *   q and k are then rounded to fp16 (the MFMA operand type): against fp32
 *   q/k the final state holds a norm-wise bar (1e-3 relative), the
 *   elementwise 1e-3 |ref| + 1e-6 only against the same rounded q and k.
 *   items_per_wg: -1 lets the launcher choose the schedule; 0 is one
 *     (sequence, v-head) item per workgroup, longest sequence first; 1..64
 *     deals the items in runs priced by their tokens to ceil(N Hv /
 *     items_per_wg) workgroups, each walking its run as one chunk stream.
 *   spin_limit: bound of the kernel's internal waits in sleep iterations,
 *     0..2^22 (-1: 2^22); 0 forces the give-up path described above (tests).
 * GDN_ERR_ARG for unknown flags or an option out of range.
 */
#define GDN_PREFILL_ZERO_INIT 1
#define GDN_PREFILL_ACCUM_STATE 2
#define GDN_PREFILL_ACCUM_OUT 4
int gdn_chunk_prefill_ex(const gdn_tensor* q, const gdn_tensor* k, const gdn_tensor* v,
                         const gdn_tensor* g, const gdn_tensor* beta, gdn_tensor* state,
                         const gdn_tensor* state_indices, const gdn_tensor* cu_seqlens,
                         gdn_tensor* out, float scale, int32_t chunk_size, int32_t flags,
                         int32_t items_per_wg, int32_t spin_limit, void* stream);

/*
 * Varlen depthwise causal conv1d + SiLU with conv-state carry-in/out
 * (replaces causal_conv1d_fn, ops/causal_conv1d.py:221-273).
 *   x          : (T, D) bf16|f16|f32, last stride 1
 *   weight     : (D, W) same dtype as x or f32, any strides, 2 <= W <= 6
 *   conv_state : (S, W-1, D) f32|bf16|f16, last stride 1; rows oldest first
 *   conv_state_indices : (N,) i32|i64
 *   cu_seqlens : (N+1,) i32|i64
 *   out        : (T, D) same dtype as x, last stride 1
 * y_t = silu(sum_j w[:, j] * xt[t + j]) over xt = [conv_state[slot]; x_seq];
 * conv_state[slot] <- last W-1 rows of xt.  D must be a multiple of 8.
 */
int causal_conv1d_varlen(const gdn_tensor* x, const gdn_tensor* weight, gdn_tensor* conv_state,
                         const gdn_tensor* conv_state_indices, const gdn_tensor* cu_seqlens,
                         gdn_tensor* out, void* stream);

/*
 * Single-token decode conv update (replaces causal_conv1d_update,
 * ops/causal_conv1d.py:434-470).
 *   x : (B, D); out : (B, D); other tensors as for causal_conv1d_varlen.
 * y = silu(sum_j w[:, j] * xt[j]) over xt = [conv_state[slot]; x_b];
 * conv_state[slot] <- xt[1:].
 */
int causal_conv1d_step(const gdn_tensor* x, const gdn_tensor* weight, gdn_tensor* conv_state,
                       const gdn_tensor* conv_state_indices, gdn_tensor* out, void* stream);

/*
 * One decode token of a whole GDN layer's recurrent part, fused: replaces
 * the decode branch of GatedDeltaNet.forward (layers/linear_attention.py:95
 * causal_conv1d_update -> :113-114 per-head L2 norm of q, k -> :89-90 gating
 * -> :119 recurrent_gated_delta_rule).
 *   mixed_qkv   (B, D) the projections before the conv, D = 2 Hk K + Hv V,
 *               channels q (Hk K) | k (Hk K) | v (Hv V); out has its dtype
 *   conv_weight (D, 4); conv_state (conv_slots, 3, D); conv_state_indices (B,)
 *   a, b        (B, Hv) gate and beta inputs; A_log, dt_bias (Hv,)
 *   state       (slots, Hv, K, V) fp32, K = V = 128; state_indices (B,)
 *   out         (B, Hv, V)
 * Per sequence: xt = [conv_state[cslot]; mixed_qkv_b], y = silu(sum_j w[:, j] xt[j]),
 * conv_state[cslot] <- xt[1:]; q, k, v = split(y); q, k <- x rsqrt(sum x^2 + 1e-6)
 * per head; g = -exp(A_log) softplus(a + dt_bias), beta = sigmoid(b); then the
 * gated delta rule step of gdn_recurrent_step with scale.  The conv output,
 * the normalised q, k and the gates stay in fp32 (no rounding to the input
 * dtype between the steps).  A padding conv slot gives a zero conv output
 * (as causal_conv1d_step does); a padding state slot gives a zero output row
 * and leaves the state untouched; the two caches are indexed independently.
 * Hv / Hk must be 1, 2 or 4; both caches need at least one slot when B > 0.
 */
int gdn_decode_step_fused(const gdn_tensor* mixed_qkv, const gdn_tensor* conv_weight, gdn_tensor* conv_state,
                          const gdn_tensor* conv_state_indices, const gdn_tensor* a, const gdn_tensor* b,
                          const gdn_tensor* A_log, const gdn_tensor* dt_bias, gdn_tensor* state,
                          const gdn_tensor* state_indices, gdn_tensor* out, int32_t num_k_heads, float scale,
                          void* stream);

/*
 * causal_conv1d_varlen, and the per-head L2 norm of the layer
 * (layers/linear_attention.py:113-114, y * rsqrt(sum y^2 + 1e-6) over each
 * 128-channel head) applied in fp32 to output channels [0, norm_channels)
 * before the one rounding to x's dtype: the q and k of the packed q|k|v
 * projection, normalised in the conv's epilogue.  norm_channels: a multiple
 * of 128, at most D.  No counterpart in the reference as one op.
 */
int causal_conv1d_varlen_qknorm(const gdn_tensor* x, const gdn_tensor* weight, gdn_tensor* conv_state,
                                const gdn_tensor* conv_state_indices, const gdn_tensor* cu_seqlens,
                                gdn_tensor* out, int64_t norm_channels, void* stream);

/*
 * Gated RMSNorm of the GDN output <- RMSNormGated, layers/norm.py:44-58 (applied
 * per v-head at layers/linear_attention.py:121):
 *   out = x * rsqrt(mean(x^2) + eps) * weight * silu(gate), fp32 math, the
 *   mean over the last dim (as the reference's, for any normalized_shape).
 * x, gate, out: (T, H, N), same dtype (fp32, bf16 or fp16), unit inner
 * stride, any N >= 1; weight: (N,) shared by the heads or (H, N) one row per
 * head, fp32, bf16 or fp16, unit inner stride.  N = 128 with a shared weight
 * and 16-byte aligned rows (the layer's v-heads) takes a vectorised kernel.
 */
int gdn_rms_norm_gated(const gdn_tensor* x, const gdn_tensor* gate, const gdn_tensor* weight, gdn_tensor* out,
                       float eps, void* stream);

/*
 * The layer's gates <- layers/linear_attention.py:89-90:
 *   g = -exp(A_log) * softplus(a + dt_bias),  beta = sigmoid(b),  fp32 math.
 * a, b: (T, H) fp32|bf16|fp16, unit inner stride; A_log, dt_bias: (H,);
 * g, beta: (T, H) fp32 outputs.
 */
int gdn_gating(const gdn_tensor* a, const gdn_tensor* b, const gdn_tensor* A_log, const gdn_tensor* dt_bias,
               gdn_tensor* g, gdn_tensor* beta, void* stream);

/*
 * Full attention of the hybrid stack's attention layers (GQA: query head h
 * reads kv head h / (Hq / Hkv)); bf16 or fp16 throughout, fp32 softmax, P
 * rounded to the input dtype before P V.  Head dim D = 64, 128 or 256 (the
 * same for q, k and v); unit inner strides and 16-byte aligned rows.
 *
 * flash_attention_varlen <- flash_attention_prefill, ops/full_attention.py:114-173
 *   q (T, Hq, D), k, v (T, Hkv, D), out (T, Hq, D), cu_seqlens (N+1,).
 *   Per sequence, query i attends keys 0..i (causal != 0) or all the
 *   sequence's keys.  max_seqlen must be at least the longest sequence, as
 *   the reference requires; here it only sizes the range check (the grid
 *   covers every sequence's query tiles).  GDN_ERR_RANGE when
 *   max(max_seqlen, 64) rows of k or v span 2^31 bytes or more.
 */
int flash_attention_varlen(const gdn_tensor* q, const gdn_tensor* k, const gdn_tensor* v,
                           const gdn_tensor* cu_seqlens, gdn_tensor* out, int64_t max_seqlen, float scale,
                           int32_t causal, void* stream);

/*
 * paged_attention_prefill <- paged_flash_attention_prefill, ops/full_attention.py:454-512
 *   q, out (T, Hq, D); k_cache, v_cache (num_blocks, page, Hkv, D);
 *   block_tables (N, max_blocks) i32|i64; context_lens (N,); cu_seqlens (N+1,).
 *   Query i of sequence n sits at position context_lens[n] - len_n + i and
 *   attends causally to cached keys 0..position, key j at slot j % page of
 *   block block_tables[n][j / page].  A query with no visible key gives a
 *   zero row; table entries outside [0, num_blocks) read as zero keys (never
 *   out of bounds).  The reference's block_m_indices work list is not needed.
 *   GDN_ERR_RANGE when one page of one kv head spans 2^31 bytes or more, or
 *   max_blocks * page >= 2^31.
 */
int paged_attention_prefill(const gdn_tensor* q, const gdn_tensor* k_cache, const gdn_tensor* v_cache,
                            const gdn_tensor* block_tables, const gdn_tensor* context_lens,
                            const gdn_tensor* cu_seqlens, gdn_tensor* out, int64_t max_seqlen, float scale,
                            void* stream);

/*
 * paged_attention_decode <- paged_flash_attention_decode, ops/full_attention.py:282-335
 *   q, out (B, Hq, D): one query per sequence, at position context_lens[b] - 1;
 *   caches and block_tables (B, max_blocks) as above.  num_splits 1..256.
 *   One split: a wave per (sequence, kv head) streams the whole sequence.
 *   num_splits > 1: the batch is dealt over U = B * (num_splits - 1) units of
 *   equal price, sequence b costing ceil(L_b / 16) 16-key tiles plus 2 (0
 *   when L_b = 0), so every unit streams about the same number of keys
 *   whatever the lengths; a unit may hold the end of one sequence and the
 *   start of the next, and the pieces are merged by a second launch.  The
 *   sequences' total price must stay below 2^31: B * (ceil(max_blocks * page
 *   / 16) + 2) >= 2^31 returns GDN_ERR_RANGE.  With num_splits > 1,
 *   workspace is an fp32 1-D tensor of at least
 *   paged_attention_decode_workspace_size(B, Hq, D, num_splits) elements
 *   (16-byte aligned), overwritten: B * num_splits * Hq * (D + 4) partials
 *   (one slot per piece; a piece is a (sequence, unit) pair) and the B + 1
 *   price prefix.  context_lens[b] = 0 gives a zero row.
 */
int64_t paged_attention_decode_workspace_size(int64_t num_seqs, int64_t num_q_heads, int64_t head_dim,
                                              int32_t num_splits);
int paged_attention_decode(const gdn_tensor* q, const gdn_tensor* k_cache, const gdn_tensor* v_cache,
                           const gdn_tensor* block_tables, const gdn_tensor* context_lens, gdn_tensor* out,
                           gdn_tensor* workspace, int32_t num_splits, float scale, void* stream);

/*
 * paged_attention_decode without a workspace argument and without any
 * allocation: the split partials live in a library-owned static device
 * array of GDN_DECODE_SCRATCH_FLOATS fp32 values (32 MiB, one copy on every
 * GPU the library runs on, held until the process ends).  No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments and results as paged_attention_decode with the
 * same num_splits; returns GDN_ERR_SCRATCH (nothing launched) when
 * paged_attention_decode_workspace_size(B, Hq, D, num_splits) exceeds
 * GDN_DECODE_SCRATCH_FLOATS.  Every call on one GPU shares that GPU's array:
 * calls that overlap in time on one GPU (two streams, two threads) race and
 * must be ordered by the caller.  The first call on a device looks the
 * array's address up (hipGetSymbolAddress) with that device current.
 */
#define GDN_DECODE_SCRATCH_FLOATS (8 * 1024 * 1024)
int paged_attention_decode_noalloc(const gdn_tensor* q, const gdn_tensor* k_cache, const gdn_tensor* v_cache,
                                   const gdn_tensor* block_tables, const gdn_tensor* context_lens, gdn_tensor* out,
                                   int32_t num_splits, float scale, void* stream);

/*
 * Measurement utility, no counterpart in the reference: copies nbytes (a
 * multiple of 16; both pointers 16-byte aligned) from src to dst with a plain
 * streaming kernel (16-byte non-temporal loads and stores, grid-stride loop
 * over `blocks` workgroups of 256 threads, 0 = one pass).  The benchmark's
 * measured HBM ceiling and the calibration of the HBM byte counters.
 */
int gdn_hbm_copy(const void* src, void* dst, int64_t nbytes, int32_t blocks, void* stream);

/* Text for any return code of this library. */
const char* gdn_strerror(int code);

/* GDN_ABI_VERSION of the built library. */
int gdn_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* GDN_HIP_H_ */
