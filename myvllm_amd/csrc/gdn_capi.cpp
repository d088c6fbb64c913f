// C ABI of libgdn_hip.so: host-side validation and dispatch.
//
// Every check runs before any HIP call, so a malformed call returns a
// negative code without touching the device (and these paths are testable on
// a machine with no GPU).  The reference ops validate nothing beyond a few
// asserts (ops/gated_delta_rule/solve_tril.py:98, ops/gated_delta_rule/h.py:211).
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <stdint.h>

#include "../../include/gdn_hip.h"

hipError_t gdn_recurrent_step_launch(const gdn_tensor* q, const gdn_tensor* k, const gdn_tensor* v,
                                     const gdn_tensor* g, const gdn_tensor* beta, gdn_tensor* state,
                                     const gdn_tensor* idx, gdn_tensor* out, float scale, hipStream_t st);
hipError_t gdn_chunk_prefill_launch(const gdn_tensor* q, const gdn_tensor* k, const gdn_tensor* v,
                                    const gdn_tensor* g, const gdn_tensor* beta, gdn_tensor* state,
                                    const gdn_tensor* idx, const gdn_tensor* cu, gdn_tensor* out, float scale,
                                    int32_t flags, int32_t spin_limit, int32_t items_per_wg, hipStream_t st);
hipError_t causal_conv1d_varlen_launch(const gdn_tensor* x, const gdn_tensor* w, gdn_tensor* cs,
                                       const gdn_tensor* idx, const gdn_tensor* cu, gdn_tensor* out,
                                       int64_t norm_ch, hipStream_t st);
hipError_t gdn_rms_norm_gated_launch(const gdn_tensor* x, const gdn_tensor* gate, const gdn_tensor* w,
                                     gdn_tensor* out, float eps, bool fast, hipStream_t st);
hipError_t gdn_gating_launch(const gdn_tensor* ga, const gdn_tensor* gb, const gdn_tensor* A_log,
                             const gdn_tensor* dt_bias, gdn_tensor* g, gdn_tensor* beta, hipStream_t st);
hipError_t causal_conv1d_step_launch(const gdn_tensor* x, const gdn_tensor* w, gdn_tensor* cs,
                                     const gdn_tensor* idx, gdn_tensor* out, hipStream_t st);
hipError_t gdn_decode_fused_launch(const gdn_tensor* x, const gdn_tensor* w, gdn_tensor* cs, const gdn_tensor* cidx,
                                   const gdn_tensor* ga, const gdn_tensor* gb, const gdn_tensor* A_log,
                                   const gdn_tensor* dt_bias, gdn_tensor* state, const gdn_tensor* sidx,
                                   gdn_tensor* out, int32_t Hk, float scale, hipStream_t st);

hipError_t attn_varlen_prefill_launch(const gdn_tensor* q, const gdn_tensor* k, const gdn_tensor* v,
                                      const gdn_tensor* cu, gdn_tensor* out, int64_t max_seqlen, float scale,
                                      int causal, hipStream_t st);
hipError_t attn_paged_prefill_launch(const gdn_tensor* q, const gdn_tensor* kc, const gdn_tensor* vc,
                                     const gdn_tensor* tab, const gdn_tensor* ctx, const gdn_tensor* cu,
                                     gdn_tensor* out, int64_t max_seqlen, float scale, hipStream_t st);
hipError_t attn_paged_decode_launch(const gdn_tensor* q, const gdn_tensor* kc, const gdn_tensor* vc,
                                    const gdn_tensor* tab, const gdn_tensor* ctx, gdn_tensor* out, float* workspace,
                                    int32_t splits, float scale, hipStream_t st);
hipError_t attn_decode_scratch(hipStream_t st, float** ptr);
int32_t attn_decode_start_price();
hipError_t hbm_stream_copy_launch(const void* src, void* dst, int64_t nbytes, int32_t blocks, hipStream_t st);

#define GDN_EXPORT extern "C" __attribute__((visibility("default")))

namespace {

constexpr int64_t kMaxGrid = 2147483647;

int64_t numel(const gdn_tensor* t) {
  int64_t n = 1;
  for (int i = 0; i < t->ndim; ++i) n *= t->shape[i];
  return n;
}

int elem_size(int dt) {
  switch (dt) {
    case GDN_DTYPE_F32: case GDN_DTYPE_I32: return 4;
    case GDN_DTYPE_BF16: case GDN_DTYPE_F16: return 2;
    case GDN_DTYPE_I64: return 8;
    default: return 0;
  }
}

bool is_float(int dt) { return dt == GDN_DTYPE_F32 || dt == GDN_DTYPE_BF16 || dt == GDN_DTYPE_F16; }
bool is_index(int dt) { return dt == GDN_DTYPE_I32 || dt == GDN_DTYPE_I64; }

// descriptor present, rank as expected, sizes non-negative, data present when non-empty
int check_desc(const gdn_tensor* t, int ndim) {
  if (!t) return GDN_ERR_NULL;
  if (t->ndim != ndim) return GDN_ERR_NDIM;
  for (int i = 0; i < ndim; ++i)
    if (t->shape[i] < 0) return GDN_ERR_SHAPE;
  if (elem_size(t->dtype) == 0) return GDN_ERR_DTYPE;
  if (numel(t) > 0 && !t->data) return GDN_ERR_NULL;
  return GDN_OK;
}

bool aligned(const gdn_tensor* t, int bytes) {
  return (reinterpret_cast<uintptr_t>(t->data) % (uintptr_t)bytes) == 0;
}

// 16-byte vectors along the last dim: pointer aligned and every outer stride a
// whole number of vectors.
bool vec_ok(const gdn_tensor* t, int vec_bytes) {
  const int es = elem_size(t->dtype);
  if (!aligned(t, vec_bytes)) return false;
  for (int i = 0; i + 1 < t->ndim; ++i)
    if ((t->stride[i] * es) % vec_bytes != 0) return false;
  return true;
}

#define GDN_TRY(expr)          \
  do {                         \
    int rc_ = (expr);          \
    if (rc_ != GDN_OK) return rc_; \
  } while (0)

int check_recurrent(const gdn_tensor* q, const gdn_tensor* k, const gdn_tensor* v, const gdn_tensor* g,
                    const gdn_tensor* beta, const gdn_tensor* state, const gdn_tensor* idx,
                    const gdn_tensor* out, const gdn_tensor* cu, bool prefill, bool f32_out = false) {
  GDN_TRY(check_desc(q, 3));
  GDN_TRY(check_desc(k, 3));
  GDN_TRY(check_desc(v, 3));
  GDN_TRY(check_desc(g, 2));
  GDN_TRY(check_desc(beta, 2));
  GDN_TRY(check_desc(state, 4));
  GDN_TRY(check_desc(idx, 1));
  GDN_TRY(check_desc(out, 3));
  if (prefill) GDN_TRY(check_desc(cu, 1));

  const int64_t T = q->shape[0], Hk = q->shape[1], K = q->shape[2];
  const int64_t Hv = v->shape[1], V = v->shape[2];
  for (int i = 0; i < 3; ++i)
    if (k->shape[i] != q->shape[i]) return GDN_ERR_SHAPE;
  if (v->shape[0] != T || out->shape[0] != T || out->shape[1] != Hv || out->shape[2] != V) return GDN_ERR_SHAPE;
  if (g->shape[0] != T || g->shape[1] != Hv || beta->shape[0] != T || beta->shape[1] != Hv) return GDN_ERR_SHAPE;
  if (state->shape[1] != Hv || state->shape[2] != K || state->shape[3] != V) return GDN_ERR_SHAPE;
  if (prefill) {
    if (cu->shape[0] < 1 || idx->shape[0] != cu->shape[0] - 1) return GDN_ERR_SHAPE;
  } else {
    if (idx->shape[0] != T) return GDN_ERR_SHAPE;
  }
  if (Hk <= 0 || Hv % Hk != 0) return GDN_ERR_HEADS;

  // dtypes
  if (k->dtype != q->dtype || v->dtype != q->dtype) return GDN_ERR_DTYPE;
  if (f32_out ? (q->dtype != GDN_DTYPE_F16 || out->dtype != GDN_DTYPE_F32) : out->dtype != v->dtype)
    return GDN_ERR_DTYPE;
  if (!is_float(q->dtype) || !is_float(g->dtype) || !is_float(beta->dtype)) return GDN_ERR_DTYPE;
  if (state->dtype != GDN_DTYPE_F32 || !is_index(idx->dtype)) return GDN_ERR_DTYPE;
  if (prefill && ((q->dtype != GDN_DTYPE_BF16 && q->dtype != GDN_DTYPE_F16) || g->dtype != GDN_DTYPE_F32 ||
                  !is_index(cu->dtype)))
    return GDN_ERR_DTYPE;

  // head dims
  if (prefill) {
    // multiples of 8 up to 128 (16-byte rows); below 128 the kernel pads with zeros
    if (K < 8 || K > 128 || K % 8 != 0 || V < 8 || V > 128 || V % 8 != 0) return GDN_ERR_HEAD_DIM;
  } else {
    // multiples of 8 up to 256 (64 x 64, 128 x 128 and 256 x 256 have their own
    // kernels, others run zero-padded in the 128 x 128 or the 256 x 256 one)
    if (K < 8 || K > 256 || K % 8 != 0 || V < 8 || V > 256 || V % 8 != 0) return GDN_ERR_HEAD_DIM;
  }

  // strides
  if (q->stride[2] != 1 || k->stride[2] != 1 || v->stride[2] != 1 || out->stride[2] != 1) return GDN_ERR_STRIDE;
  if (state->stride[3] != 1 || state->stride[2] != V) return GDN_ERR_STRIDE;
  if (idx->stride[0] != 1 || (prefill && cu->stride[0] != 1)) return GDN_ERR_STRIDE;

  // alignment: fp32 state rows as 16-byte vectors; prefill q/k/v/out as 16-byte vectors
  if (T > 0 && !vec_ok(state, 16)) return GDN_ERR_ALIGN;
  if (prefill && T > 0) {
    if (!vec_ok(q, 16) || !vec_ok(k, 16) || !vec_ok(v, 16) || !vec_ok(out, 16)) return GDN_ERR_ALIGN;
  }

  // index ranges
  if (prefill) {
    if (idx->shape[0] * Hv > kMaxGrid || T > kMaxGrid) return GDN_ERR_RANGE;
    // the prefill kernel addresses the rows of a 64-token chunk with 32-bit offsets
    const int64_t kMaxTokenStride = int64_t(1) << 24;
    if (q->stride[0] > kMaxTokenStride || k->stride[0] > kMaxTokenStride || v->stride[0] > kMaxTokenStride ||
        out->stride[0] > kMaxTokenStride)
      return GDN_ERR_RANGE;
  } else {
    if (T * Hv > kMaxGrid) return GDN_ERR_RANGE;
  }
  return GDN_OK;
}

int check_conv(const gdn_tensor* x, const gdn_tensor* w, const gdn_tensor* cs, const gdn_tensor* idx,
               const gdn_tensor* cu, const gdn_tensor* out, bool varlen) {
  GDN_TRY(check_desc(x, 2));
  GDN_TRY(check_desc(w, 2));
  GDN_TRY(check_desc(cs, 3));
  GDN_TRY(check_desc(idx, 1));
  GDN_TRY(check_desc(out, 2));
  if (varlen) GDN_TRY(check_desc(cu, 1));

  const int64_t T = x->shape[0], D = x->shape[1], W = w->shape[1];
  if (W < 2 || W > 6) return GDN_ERR_CONV_WIDTH;
  if (w->shape[0] != D || cs->shape[1] != W - 1 || cs->shape[2] != D) return GDN_ERR_SHAPE;
  if (out->shape[0] != T || out->shape[1] != D) return GDN_ERR_SHAPE;
  if (varlen) {
    if (cu->shape[0] < 1 || idx->shape[0] != cu->shape[0] - 1) return GDN_ERR_SHAPE;
  } else {
    if (idx->shape[0] != T) return GDN_ERR_SHAPE;
  }
  if (D % 8 != 0) return GDN_ERR_SHAPE;

  if (!is_float(x->dtype) || out->dtype != x->dtype) return GDN_ERR_DTYPE;
  if (w->dtype != x->dtype && w->dtype != GDN_DTYPE_F32) return GDN_ERR_DTYPE;
  if (cs->dtype != x->dtype && cs->dtype != GDN_DTYPE_F32) return GDN_ERR_DTYPE;
  if (!is_index(idx->dtype) || (varlen && !is_index(cu->dtype))) return GDN_ERR_DTYPE;

  if (x->stride[1] != 1 || out->stride[1] != 1 || cs->stride[2] != 1) return GDN_ERR_STRIDE;
  if (idx->stride[0] != 1 || (varlen && cu->stride[0] != 1)) return GDN_ERR_STRIDE;

  if (T > 0 && D > 0) {
    if (!vec_ok(x, 16) || !vec_ok(out, 16)) return GDN_ERR_ALIGN;
    if (!vec_ok(cs, 16)) return GDN_ERR_ALIGN;
  }
  if (T > kMaxGrid || D / 8 > kMaxGrid) return GDN_ERR_RANGE;
  // the varlen kernel addresses the rows of a 64-token tile with 32-bit byte offsets
  if (x->stride[0] > (int64_t(1) << 23) || out->stride[0] > (int64_t(1) << 23)) return GDN_ERR_RANGE;
  return GDN_OK;
}

int check_fused(const gdn_tensor* x, const gdn_tensor* w, const gdn_tensor* cs, const gdn_tensor* cidx,
                const gdn_tensor* ga, const gdn_tensor* gb, const gdn_tensor* A_log, const gdn_tensor* dt_bias,
                const gdn_tensor* state, const gdn_tensor* sidx, const gdn_tensor* out, int32_t Hk) {
  GDN_TRY(check_desc(x, 2));
  GDN_TRY(check_desc(w, 2));
  GDN_TRY(check_desc(cs, 3));
  GDN_TRY(check_desc(cidx, 1));
  GDN_TRY(check_desc(ga, 2));
  GDN_TRY(check_desc(gb, 2));
  GDN_TRY(check_desc(A_log, 1));
  GDN_TRY(check_desc(dt_bias, 1));
  GDN_TRY(check_desc(state, 4));
  GDN_TRY(check_desc(sidx, 1));
  GDN_TRY(check_desc(out, 3));

  const int64_t B = x->shape[0], D = x->shape[1];
  const int64_t Hv = state->shape[1], K = state->shape[2], V = state->shape[3];
  if (w->shape[1] != 4) return GDN_ERR_CONV_WIDTH;
  if (K != 128 || V != 128) return GDN_ERR_HEAD_DIM;
  if (Hk <= 0 || Hv % Hk != 0) return GDN_ERR_HEADS;
  const int64_t r = Hv / Hk;
  if (r != 1 && r != 2 && r != 4) return GDN_ERR_HEADS;
  if (D != 2 * Hk * K + Hv * V) return GDN_ERR_SHAPE;
  if (w->shape[0] != D || cs->shape[1] != 3 || cs->shape[2] != D) return GDN_ERR_SHAPE;
  if (cidx->shape[0] != B || sidx->shape[0] != B) return GDN_ERR_SHAPE;
  if (ga->shape[0] != B || ga->shape[1] != Hv || gb->shape[0] != B || gb->shape[1] != Hv) return GDN_ERR_SHAPE;
  if (A_log->shape[0] != Hv || dt_bias->shape[0] != Hv) return GDN_ERR_SHAPE;
  if (out->shape[0] != B || out->shape[1] != Hv || out->shape[2] != V) return GDN_ERR_SHAPE;
  // padding rows still read slot 0 of each cache (branch-free loads), so a
  // non-empty batch needs a non-empty cache
  if (B > 0 && (cs->shape[0] < 1 || state->shape[0] < 1)) return GDN_ERR_SHAPE;

  if (!is_float(x->dtype) || out->dtype != x->dtype) return GDN_ERR_DTYPE;
  if (!is_float(w->dtype) || !is_float(cs->dtype) || !is_float(ga->dtype) || !is_float(gb->dtype) ||
      !is_float(A_log->dtype) || !is_float(dt_bias->dtype))
    return GDN_ERR_DTYPE;
  if (state->dtype != GDN_DTYPE_F32 || !is_index(cidx->dtype) || !is_index(sidx->dtype)) return GDN_ERR_DTYPE;

  if (x->stride[1] != 1 || cs->stride[2] != 1 || out->stride[2] != 1) return GDN_ERR_STRIDE;
  if (state->stride[3] != 1 || state->stride[2] != V) return GDN_ERR_STRIDE;
  if (cidx->stride[0] != 1 || sidx->stride[0] != 1) return GDN_ERR_STRIDE;
  if (B > 0 && !vec_ok(state, 16)) return GDN_ERR_ALIGN;
  if (B * Hk > kMaxGrid) return GDN_ERR_RANGE;
  return GDN_OK;
}

int launch_rc(hipError_t e) { return e == hipSuccess ? GDN_OK : (int)e; }

// Bound of the prefill kernel's internal waits between its wave roles (sleep
// iterations; never reached when the pipeline is correct).
constexpr int32_t kPrefillSpinLimit = 1 << 22;

constexpr int64_t kMaxGridYZ = 65535;
constexpr int32_t kMaxDecodeSplits = 256;

// q / out (rows, Hq, D) with the kv tensors' head count and head dim: bf16 or
// fp16 throughout, D = 64, 128 or 256, unit inner strides, 16-byte rows.
int check_attn_qo(const gdn_tensor* q, const gdn_tensor* out, const gdn_tensor* kv0, const gdn_tensor* kv1,
                  int64_t Hkv) {
  const int64_t rows = q->shape[0], Hq = q->shape[1], D = q->shape[2];
  if (out->shape[0] != rows || out->shape[1] != Hq || out->shape[2] != D) return GDN_ERR_SHAPE;
  const int kd = kv0->ndim - 1;
  if (kv0->shape[kd] != D || kv1->shape[kd] != D) return GDN_ERR_SHAPE;
  if (Hkv <= 0 || Hq <= 0 || Hq % Hkv != 0) return GDN_ERR_HEADS;
  if (q->dtype != GDN_DTYPE_BF16 && q->dtype != GDN_DTYPE_F16) return GDN_ERR_DTYPE;
  if (kv0->dtype != q->dtype || kv1->dtype != q->dtype || out->dtype != q->dtype) return GDN_ERR_DTYPE;
  if (D != 64 && D != 128 && D != 256) return GDN_ERR_HEAD_DIM;
  if (q->stride[2] != 1 || out->stride[2] != 1 || kv0->stride[kd] != 1 || kv1->stride[kd] != 1)
    return GDN_ERR_STRIDE;
  if (numel(q) > 0 && (!vec_ok(q, 16) || !vec_ok(out, 16))) return GDN_ERR_ALIGN;
  if (numel(kv0) > 0 && (!vec_ok(kv0, 16) || !vec_ok(kv1, 16))) return GDN_ERR_ALIGN;
  return GDN_OK;
}

// paged caches (blocks, page, Hkv, D), block table (N, cols), context lengths (N,)
int check_paged(const gdn_tensor* kc, const gdn_tensor* vc, const gdn_tensor* tab, const gdn_tensor* ctx,
                int64_t N) {
  GDN_TRY(check_desc(kc, 4));
  GDN_TRY(check_desc(vc, 4));
  GDN_TRY(check_desc(tab, 2));
  GDN_TRY(check_desc(ctx, 1));
  for (int i = 0; i < 4; ++i)
    if (vc->shape[i] != kc->shape[i]) return GDN_ERR_SHAPE;
  if (tab->shape[0] != N || ctx->shape[0] != N) return GDN_ERR_SHAPE;
  if (kc->shape[1] <= 0 || kc->shape[1] > INT32_MAX) return GDN_ERR_SHAPE;
  if (!is_index(tab->dtype) || !is_index(ctx->dtype)) return GDN_ERR_DTYPE;
  if (tab->stride[1] != 1 || ctx->stride[0] != 1) return GDN_ERR_STRIDE;
  return GDN_OK;
}

}  // namespace

GDN_EXPORT int gdn_abi_version(void) { return GDN_ABI_VERSION; }

GDN_EXPORT const char* gdn_strerror(int code) {
  switch (code) {
    case GDN_OK: return "success";
    case GDN_ERR_NULL: return "missing tensor descriptor or data pointer";
    case GDN_ERR_NDIM: return "tensor has the wrong number of dimensions";
    case GDN_ERR_SHAPE: return "tensor shapes are inconsistent";
    case GDN_ERR_DTYPE: return "unsupported tensor dtype";
    case GDN_ERR_STRIDE: return "unsupported strides (innermost dims must be contiguous)";
    case GDN_ERR_HEADS: return "num_v_heads must be a positive multiple of num_k_heads";
    case GDN_ERR_HEAD_DIM: return "unsupported head dims";
    case GDN_ERR_CHUNK: return "unsupported chunk size (64 required)";
    case GDN_ERR_ALIGN: return "pointer or stride misaligned for 16-byte vector access";
    case GDN_ERR_CONV_WIDTH: return "conv width must be in [2, 6]";
    case GDN_ERR_RANGE: return "size exceeds the kernels' index range";
    case GDN_ERR_ARG: return "an option argument is out of range";
    case GDN_ERR_SCRATCH: return "the call needs more split scratch than the library's static array holds "
                                 "(GDN_DECODE_SCRATCH_FLOATS fp32 values); use fewer splits or the workspace entry";
    default: break;
  }
  if (code > 0) return hipGetErrorString((hipError_t)code);
  return "unknown error code";
}

GDN_EXPORT int gdn_recurrent_step(const gdn_tensor* q, const gdn_tensor* k, const gdn_tensor* v,
                                  const gdn_tensor* g, const gdn_tensor* beta, gdn_tensor* state,
                                  const gdn_tensor* state_indices, gdn_tensor* out, float scale, void* stream) {
  GDN_TRY(check_recurrent(q, k, v, g, beta, state, state_indices, out, nullptr, false));
  return launch_rc(gdn_recurrent_step_launch(q, k, v, g, beta, state, state_indices, out, scale,
                                             reinterpret_cast<hipStream_t>(stream)));
}

GDN_EXPORT int gdn_chunk_prefill(const gdn_tensor* q, const gdn_tensor* k, const gdn_tensor* v,
                                 const gdn_tensor* g, const gdn_tensor* beta, gdn_tensor* state,
                                 const gdn_tensor* state_indices, const gdn_tensor* cu_seqlens,
                                 gdn_tensor* out, float scale, int32_t chunk_size, void* stream) {
  if (chunk_size != 64) return GDN_ERR_CHUNK;
  GDN_TRY(check_recurrent(q, k, v, g, beta, state, state_indices, out, cu_seqlens, true));
  return launch_rc(gdn_chunk_prefill_launch(q, k, v, g, beta, state, state_indices, cu_seqlens, out, scale, 0,
                                            kPrefillSpinLimit, -1, reinterpret_cast<hipStream_t>(stream)));
}

GDN_EXPORT int gdn_chunk_prefill_ex(const gdn_tensor* q, const gdn_tensor* k, const gdn_tensor* v,
                                    const gdn_tensor* g, const gdn_tensor* beta, gdn_tensor* state,
                                    const gdn_tensor* state_indices, const gdn_tensor* cu_seqlens,
                                    gdn_tensor* out, float scale, int32_t chunk_size, int32_t flags,
                                    int32_t items_per_wg, int32_t spin_limit, void* stream) {
  if (chunk_size != 64) return GDN_ERR_CHUNK;
  constexpr int32_t kKnown = GDN_PREFILL_ZERO_INIT | GDN_PREFILL_ACCUM_STATE | GDN_PREFILL_ACCUM_OUT;
  if ((flags & ~kKnown) != 0 || items_per_wg < -1 || items_per_wg > 64 || spin_limit < -1 ||
      spin_limit > kPrefillSpinLimit)
    return GDN_ERR_ARG;
  const bool f32_out = out && out->dtype == GDN_DTYPE_F32;
  if ((flags & GDN_PREFILL_ACCUM_OUT) && !f32_out) return GDN_ERR_DTYPE;
  GDN_TRY(check_recurrent(q, k, v, g, beta, state, state_indices, out, cu_seqlens, true, f32_out));
  return launch_rc(gdn_chunk_prefill_launch(q, k, v, g, beta, state, state_indices, cu_seqlens, out, scale, flags,
                                            spin_limit < 0 ? kPrefillSpinLimit : spin_limit, items_per_wg,
                                            reinterpret_cast<hipStream_t>(stream)));
}

GDN_EXPORT int causal_conv1d_varlen(const gdn_tensor* x, const gdn_tensor* weight, gdn_tensor* conv_state,
                                    const gdn_tensor* conv_state_indices, const gdn_tensor* cu_seqlens,
                                    gdn_tensor* out, void* stream) {
  GDN_TRY(check_conv(x, weight, conv_state, conv_state_indices, cu_seqlens, out, true));
  return launch_rc(causal_conv1d_varlen_launch(x, weight, conv_state, conv_state_indices, cu_seqlens, out, 0,
                                               reinterpret_cast<hipStream_t>(stream)));
}

GDN_EXPORT int causal_conv1d_step(const gdn_tensor* x, const gdn_tensor* weight, gdn_tensor* conv_state,
                                  const gdn_tensor* conv_state_indices, gdn_tensor* out, void* stream) {
  GDN_TRY(check_conv(x, weight, conv_state, conv_state_indices, nullptr, out, false));
  return launch_rc(causal_conv1d_step_launch(x, weight, conv_state, conv_state_indices, out,
                                             reinterpret_cast<hipStream_t>(stream)));
}

GDN_EXPORT int gdn_decode_step_fused(const gdn_tensor* mixed_qkv, const gdn_tensor* conv_weight,
                                     gdn_tensor* conv_state, const gdn_tensor* conv_state_indices,
                                     const gdn_tensor* a, const gdn_tensor* b, const gdn_tensor* A_log,
                                     const gdn_tensor* dt_bias, gdn_tensor* state, const gdn_tensor* state_indices,
                                     gdn_tensor* out, int32_t num_k_heads, float scale, void* stream) {
  GDN_TRY(check_fused(mixed_qkv, conv_weight, conv_state, conv_state_indices, a, b, A_log, dt_bias, state,
                      state_indices, out, num_k_heads));
  return launch_rc(gdn_decode_fused_launch(mixed_qkv, conv_weight, conv_state, conv_state_indices, a, b, A_log,
                                           dt_bias, state, state_indices, out, num_k_heads, scale,
                                           reinterpret_cast<hipStream_t>(stream)));
}

GDN_EXPORT int causal_conv1d_varlen_qknorm(const gdn_tensor* x, const gdn_tensor* weight, gdn_tensor* conv_state,
                                           const gdn_tensor* conv_state_indices, const gdn_tensor* cu_seqlens,
                                           gdn_tensor* out, int64_t norm_channels, void* stream) {
  GDN_TRY(check_conv(x, weight, conv_state, conv_state_indices, cu_seqlens, out, true));
  if (norm_channels < 0 || norm_channels % 128 != 0 || norm_channels > x->shape[1]) return GDN_ERR_SHAPE;
  return launch_rc(causal_conv1d_varlen_launch(x, weight, conv_state, conv_state_indices, cu_seqlens, out,
                                               norm_channels, reinterpret_cast<hipStream_t>(stream)));
}

GDN_EXPORT int gdn_rms_norm_gated(const gdn_tensor* x, const gdn_tensor* gate, const gdn_tensor* weight,
                                  gdn_tensor* out, float eps, void* stream) {
  GDN_TRY(check_desc(x, 3));
  GDN_TRY(check_desc(gate, 3));
  if (!weight) return GDN_ERR_NULL;
  GDN_TRY(check_desc(weight, weight->ndim == 2 ? 2 : 1));
  GDN_TRY(check_desc(out, 3));
  for (int i = 0; i < 3; ++i)
    if (gate->shape[i] != x->shape[i] || out->shape[i] != x->shape[i]) return GDN_ERR_SHAPE;
  const int64_t H = x->shape[1], N = x->shape[2];
  // weight: one row of N shared by every head, or one row per head (H, N)
  if (weight->ndim == 1 ? weight->shape[0] != N : (weight->shape[0] != H || weight->shape[1] != N))
    return GDN_ERR_SHAPE;
  if (!is_float(x->dtype) || out->dtype != x->dtype || gate->dtype != x->dtype || !is_float(weight->dtype))
    return GDN_ERR_DTYPE;
  if (x->stride[2] != 1 || gate->stride[2] != 1 || out->stride[2] != 1 || weight->stride[weight->ndim - 1] != 1)
    return GDN_ERR_STRIDE;
  if (x->shape[0] * H > kMaxGrid * 4) return GDN_ERR_RANGE;
  // 128-element rows with one weight row and 16-byte aligned rows: the fast kernel
  const bool fast = N == 128 && weight->ndim == 1 &&
                    (numel(x) == 0 || (vec_ok(x, 16) && vec_ok(gate, 16) && vec_ok(out, 16)));
  return launch_rc(gdn_rms_norm_gated_launch(x, gate, weight, out, eps, fast, reinterpret_cast<hipStream_t>(stream)));
}

GDN_EXPORT int gdn_gating(const gdn_tensor* a, const gdn_tensor* b, const gdn_tensor* A_log, const gdn_tensor* dt_bias,
                          gdn_tensor* g, gdn_tensor* beta, void* stream) {
  GDN_TRY(check_desc(a, 2));
  GDN_TRY(check_desc(b, 2));
  GDN_TRY(check_desc(A_log, 1));
  GDN_TRY(check_desc(dt_bias, 1));
  GDN_TRY(check_desc(g, 2));
  GDN_TRY(check_desc(beta, 2));
  const int64_t T = a->shape[0], H = a->shape[1];
  if (b->shape[0] != T || b->shape[1] != H || g->shape[0] != T || g->shape[1] != H || beta->shape[0] != T ||
      beta->shape[1] != H || A_log->shape[0] != H || dt_bias->shape[0] != H)
    return GDN_ERR_SHAPE;
  if (!is_float(a->dtype) || !is_float(b->dtype) || !is_float(A_log->dtype) || !is_float(dt_bias->dtype))
    return GDN_ERR_DTYPE;
  if (g->dtype != GDN_DTYPE_F32 || beta->dtype != GDN_DTYPE_F32) return GDN_ERR_DTYPE;
  if (a->stride[1] != 1 || b->stride[1] != 1 || g->stride[1] != 1 || beta->stride[1] != 1 ||
      A_log->stride[0] != 1 || dt_bias->stride[0] != 1)
    return GDN_ERR_STRIDE;
  if (T * H > kMaxGrid) return GDN_ERR_RANGE;
  return launch_rc(gdn_gating_launch(a, b, A_log, dt_bias, g, beta, reinterpret_cast<hipStream_t>(stream)));
}

GDN_EXPORT int flash_attention_varlen(const gdn_tensor* q, const gdn_tensor* k, const gdn_tensor* v,
                                      const gdn_tensor* cu_seqlens, gdn_tensor* out, int64_t max_seqlen, float scale,
                                      int32_t causal, void* stream) {
  GDN_TRY(check_desc(q, 3));
  GDN_TRY(check_desc(k, 3));
  GDN_TRY(check_desc(v, 3));
  GDN_TRY(check_desc(out, 3));
  GDN_TRY(check_desc(cu_seqlens, 1));
  if (k->shape[0] != q->shape[0] || v->shape[0] != q->shape[0] || v->shape[1] != k->shape[1]) return GDN_ERR_SHAPE;
  if (cu_seqlens->shape[0] < 1 || max_seqlen < 0) return GDN_ERR_SHAPE;
  GDN_TRY(check_attn_qo(q, out, k, v, k->shape[1]));
  if (!is_index(cu_seqlens->dtype)) return GDN_ERR_DTYPE;
  if (cu_seqlens->stride[0] != 1) return GDN_ERR_STRIDE;
  const int64_t R = q->shape[1] / k->shape[1];
  const int64_t gh = R % 4 == 0 ? 4 : (R % 2 == 0 ? 2 : 1);
  if (cu_seqlens->shape[0] - 1 > kMaxGridYZ || q->shape[1] / gh > kMaxGridYZ || max_seqlen / 32 > kMaxGrid)
    return GDN_ERR_RANGE;
  // a sequence's kv rows, and a 64-row key tile of them, are addressed with
  // 32-bit byte offsets below 2^31
  const int64_t es = elem_size(k->dtype);
  if (std::max<int64_t>(max_seqlen, 64) * std::max(k->stride[0], v->stride[0]) * es >= (int64_t(1) << 31))
    return GDN_ERR_RANGE;
  return launch_rc(attn_varlen_prefill_launch(q, k, v, cu_seqlens, out, max_seqlen, scale, causal,
                                              reinterpret_cast<hipStream_t>(stream)));
}

GDN_EXPORT int paged_attention_prefill(const gdn_tensor* q, const gdn_tensor* k_cache, const gdn_tensor* v_cache,
                                       const gdn_tensor* block_tables, const gdn_tensor* context_lens,
                                       const gdn_tensor* cu_seqlens, gdn_tensor* out, int64_t max_seqlen,
                                       float scale, void* stream) {
  GDN_TRY(check_desc(q, 3));
  GDN_TRY(check_desc(out, 3));
  GDN_TRY(check_desc(cu_seqlens, 1));
  if (cu_seqlens->shape[0] < 1 || max_seqlen < 0) return GDN_ERR_SHAPE;
  const int64_t N = cu_seqlens->shape[0] - 1;
  GDN_TRY(check_paged(k_cache, v_cache, block_tables, context_lens, N));
  GDN_TRY(check_attn_qo(q, out, k_cache, v_cache, k_cache->shape[2]));
  if (!is_index(cu_seqlens->dtype)) return GDN_ERR_DTYPE;
  if (cu_seqlens->stride[0] != 1) return GDN_ERR_STRIDE;
  const int64_t R = q->shape[1] / k_cache->shape[2];
  const int64_t gh = R % 4 == 0 ? 4 : (R % 2 == 0 ? 2 : 1);
  if (N > kMaxGridYZ || q->shape[1] / gh > kMaxGridYZ || max_seqlen / 32 > kMaxGrid) return GDN_ERR_RANGE;
  // one page of one kv head is addressed with 32-bit byte offsets below 2^31,
  // key positions (at most columns x page) with 32-bit integers
  const int64_t es = elem_size(k_cache->dtype);
  if (k_cache->shape[1] * std::max(k_cache->stride[1], v_cache->stride[1]) * es >= (int64_t(1) << 31) ||
      block_tables->shape[1] * k_cache->shape[1] >= (int64_t(1) << 31))
    return GDN_ERR_RANGE;
  return launch_rc(attn_paged_prefill_launch(q, k_cache, v_cache, block_tables, context_lens, cu_seqlens, out,
                                             max_seqlen, scale, reinterpret_cast<hipStream_t>(stream)));
}

GDN_EXPORT int64_t paged_attention_decode_workspace_size(int64_t num_seqs, int64_t num_q_heads, int64_t head_dim,
                                                         int32_t num_splits) {
  if (num_seqs < 0 || num_q_heads < 0 || head_dim < 0 || num_splits <= 1) return 0;
  // B splits piece slots (B sequences + B (splits - 1) units) of Hq rows of
  // D + 4 floats, then the B + 1 int32 price prefix, rounded up to 16 bytes
  return num_seqs * (int64_t)num_splits * num_q_heads * (head_dim + 4) + (num_seqs + 1 + 3) / 4 * 4;
}

namespace {
// Checks shared by the two paged decode entries (everything but the workspace).
int check_paged_decode(const gdn_tensor* q, const gdn_tensor* k_cache, const gdn_tensor* v_cache,
                       const gdn_tensor* block_tables, const gdn_tensor* context_lens, const gdn_tensor* out,
                       int32_t num_splits) {
  GDN_TRY(check_desc(q, 3));
  GDN_TRY(check_desc(out, 3));
  const int64_t B = q->shape[0];
  GDN_TRY(check_paged(k_cache, v_cache, block_tables, context_lens, B));
  GDN_TRY(check_attn_qo(q, out, k_cache, v_cache, k_cache->shape[2]));
  if (num_splits < 1 || num_splits > kMaxDecodeSplits) return GDN_ERR_RANGE;
  const int64_t Hkv = k_cache->shape[2], R = q->shape[1] / Hkv;
  if (B > kMaxGridYZ || Hkv * ((R + 15) / 16) > kMaxGridYZ) return GDN_ERR_RANGE;
  // the split decode prices the batch (16-key tiles plus a start price per
  // sequence) in 32 bits
  if (num_splits > 1 &&
      B * ((block_tables->shape[1] * k_cache->shape[1] + 15) / 16 + attn_decode_start_price()) >= (int64_t(1) << 31))
    return GDN_ERR_RANGE;
  // one page of one kv head is addressed with 32-bit byte offsets below 2^31
  const int64_t es = elem_size(k_cache->dtype);
  if (k_cache->shape[1] * std::max(k_cache->stride[1], v_cache->stride[1]) * es >= (int64_t(1) << 31))
    return GDN_ERR_RANGE;
  return GDN_OK;
}
}  // namespace

GDN_EXPORT int paged_attention_decode(const gdn_tensor* q, const gdn_tensor* k_cache, const gdn_tensor* v_cache,
                                      const gdn_tensor* block_tables, const gdn_tensor* context_lens, gdn_tensor* out,
                                      gdn_tensor* workspace, int32_t num_splits, float scale, void* stream) {
  GDN_TRY(check_paged_decode(q, k_cache, v_cache, block_tables, context_lens, out, num_splits));
  const int64_t B = q->shape[0];
  float* ws = nullptr;
  if (num_splits > 1) {
    GDN_TRY(check_desc(workspace, 1));
    if (workspace->dtype != GDN_DTYPE_F32) return GDN_ERR_DTYPE;
    if (workspace->stride[0] != 1) return GDN_ERR_STRIDE;
    if (workspace->shape[0] < paged_attention_decode_workspace_size(B, q->shape[1], q->shape[2], num_splits))
      return GDN_ERR_SHAPE;
    if (B > 0 && !aligned(workspace, 16)) return GDN_ERR_ALIGN;
    ws = reinterpret_cast<float*>(workspace->data);
  }
  return launch_rc(attn_paged_decode_launch(q, k_cache, v_cache, block_tables, context_lens, out, ws, num_splits,
                                            scale, reinterpret_cast<hipStream_t>(stream)));
}

GDN_EXPORT int paged_attention_decode_noalloc(const gdn_tensor* q, const gdn_tensor* k_cache,
                                              const gdn_tensor* v_cache, const gdn_tensor* block_tables,
                                              const gdn_tensor* context_lens, gdn_tensor* out, int32_t num_splits,
                                              float scale, void* stream) {
  GDN_TRY(check_paged_decode(q, k_cache, v_cache, block_tables, context_lens, out, num_splits));
  const int64_t B = q->shape[0];
  float* ws = nullptr;
  if (num_splits > 1 && B > 0) {
    if (paged_attention_decode_workspace_size(B, q->shape[1], q->shape[2], num_splits) > GDN_DECODE_SCRATCH_FLOATS)
      return GDN_ERR_SCRATCH;
    const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    GDN_TRY(launch_rc(attn_decode_scratch(st, &ws)));
  }
  return launch_rc(attn_paged_decode_launch(q, k_cache, v_cache, block_tables, context_lens, out, ws, num_splits,
                                            scale, reinterpret_cast<hipStream_t>(stream)));
}

GDN_EXPORT int gdn_hbm_copy(const void* src, void* dst, int64_t nbytes, int32_t blocks, void* stream) {
  if (nbytes < 0 || nbytes % 16 != 0 || blocks < 0) return GDN_ERR_SHAPE;
  if (nbytes > 0 && (!src || !dst)) return GDN_ERR_NULL;
  if ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) % 16 != 0) return GDN_ERR_ALIGN;
  return launch_rc(hbm_stream_copy_launch(src, dst, nbytes, blocks, reinterpret_cast<hipStream_t>(stream)));
}
