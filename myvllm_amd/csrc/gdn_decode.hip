// Fused recurrent gated-delta-rule decode step (one token per sequence).
//
// Replaces the Triton kernel _fused_recurrent_gdn
// (ops/gated_delta_rule/fused_recurrent_gdn.py:6-102 in yuyifanbupt/myvllm),
// which tiles the fp32 state as 128x8 slabs (32 contiguous bytes per row).
// Here one 256-thread workgroup owns the whole K x V fp32 state of one
// (sequence, v-head): every thread streams V/4-wide rows with 16-byte loads
// (a wave reads 1 KiB contiguous per instruction), both reductions over K
// (k^T S and q^T S) are done in the same pass, and the updated state is
// written back in place, so the state crosses HBM exactly once each way
// (non-temporal loads and stores: nothing of it is reused by this launch).
//
// Math per (b, h), with S decayed first (fused_recurrent_gdn.py:96-99):
//   kS = k^T S, qS = (scale q)^T S                  (old S)
//   d  = beta (v - e^g kS)
//   o  = e^g qS + (scale q . k) d                   (= S_new^T (scale q))
//   S  = e^g S + k d^T
#include "gdn_common.h"

namespace {

struct RecurrentArgs {
  const void* q; const void* k; const void* v; const void* g; const void* beta;
  float* state; const void* idx; void* out;
  int64_t q_s0, q_s1, k_s0, k_s1, v_s0, v_s1, g_s0, g_s1, b_s0, b_s1, o_s0, o_s1;
  int64_t st_slot, st_head;
  int64_t num_slots;
  int32_t Hv, r;  // r = Hv / Hk
  int32_t g_dtype, b_dtype;
  float scale;
  bool idx64;
};

constexpr int kThreads = 256;

template <typename TIn, int K, int V>
__global__ __launch_bounds__(kThreads) void gdn_recurrent_step_kernel(RecurrentArgs a) {
  constexpr int CG = V / 4;           // float4 column groups per row
  constexpr int RG = kThreads / CG;   // row groups
  constexpr int NI = K / RG;          // rows per thread
  constexpr int WAVES = kThreads / 64;
  static_assert(kThreads % CG == 0 && K % RG == 0 && 64 % CG == 0, "shape");

  __shared__ float sq[K], sk[K], sv[V];
  __shared__ float red[WAVES][CG][9];

  const int tid = threadIdx.x;
  const int64_t b = blockIdx.x / a.Hv;
  const int h = blockIdx.x % a.Hv;
  const int kh = h / a.r;
  const int c4 = tid % CG;
  const int r0 = tid / CG;

  const int64_t slot = load_index(a.idx, b, a.idx64);
  TIn* o = reinterpret_cast<TIn*>(a.out) + b * a.o_s0 + h * a.o_s1;
  if (slot < 0 || slot >= a.num_slots) {  // padding sequence: zero output, state untouched
    if (tid < V) o[tid] = from_f32<TIn>(0.0f);
    return;
  }

  float* S = a.state + slot * a.st_slot + h * a.st_head;
  f32x4 s[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i)
    s[i] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(S + (int64_t)(r0 + RG * i) * V + 4 * c4));

  if (tid < K) {
    sq[tid] = to_f32(reinterpret_cast<const TIn*>(a.q)[b * a.q_s0 + kh * a.q_s1 + tid]) * a.scale;
    sk[tid] = to_f32(reinterpret_cast<const TIn*>(a.k)[b * a.k_s0 + kh * a.k_s1 + tid]);
  }
  if (tid >= kThreads - V) {
    const int j = tid - (kThreads - V);
    sv[j] = to_f32(reinterpret_cast<const TIn*>(a.v)[b * a.v_s0 + h * a.v_s1 + j]);
  }
  const float g = load_scalar_f32(a.g, b * a.g_s0 + h * a.g_s1, a.g_dtype);
  const float beta = load_scalar_f32(a.beta, b * a.b_s0 + h * a.b_s1, a.b_dtype);
  __syncthreads();

  // partial reductions over this thread's rows
  float pk[4] = {0.f, 0.f, 0.f, 0.f}, pq[4] = {0.f, 0.f, 0.f, 0.f}, qk = 0.f;
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const float kv = sk[r0 + RG * i];
    const float qv = sq[r0 + RG * i];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      pk[j] = fmaf(kv, s[i][j], pk[j]);
      pq[j] = fmaf(qv, s[i][j], pq[j]);
    }
    qk = fmaf(qv, kv, qk);
  }
  // reduce over row groups inside the wave (lanes with equal c4 differ by CG)
#pragma unroll
  for (int off = CG; off < 64; off <<= 1) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      pk[j] += __shfl_xor(pk[j], off, 64);
      pq[j] += __shfl_xor(pq[j], off, 64);
    }
    qk += __shfl_xor(qk, off, 64);
  }
  const int wave = tid >> 6;
  if ((tid & 63) < CG) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      red[wave][c4][j] = pk[j];
      red[wave][c4][4 + j] = pq[j];
    }
    red[wave][c4][8] = qk;
  }
  __syncthreads();
  float kS[4] = {0.f, 0.f, 0.f, 0.f}, qS[4] = {0.f, 0.f, 0.f, 0.f};
  qk = 0.f;
#pragma unroll
  for (int w = 0; w < WAVES; ++w) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      kS[j] += red[w][c4][j];
      qS[j] += red[w][c4][4 + j];
    }
    qk += red[w][c4][8];
  }

  const float eg = __expf(g);
  float d[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) d[j] = beta * (sv[4 * c4 + j] - eg * kS[j]);

#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const float kv = sk[r0 + RG * i];
    f32x4 t;
#pragma unroll
    for (int j = 0; j < 4; ++j) t[j] = fmaf(eg, s[i][j], kv * d[j]);
    __builtin_nontemporal_store(t, reinterpret_cast<f32x4*>(S + (int64_t)(r0 + RG * i) * V + 4 * c4));
  }
  if (r0 == 0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) o[4 * c4 + j] = from_f32<TIn>(fmaf(eg, qS[j], qk * d[j]));
  }
}

template <typename TIn>
hipError_t launch_dims(const RecurrentArgs& a, int K, int V, int64_t nblocks, hipStream_t st) {
  if (K == 128 && V == 128)
    gdn_recurrent_step_kernel<TIn, 128, 128><<<dim3((unsigned)nblocks), dim3(kThreads), 0, st>>>(a);
  else
    gdn_recurrent_step_kernel<TIn, 64, 64><<<dim3((unsigned)nblocks), dim3(kThreads), 0, st>>>(a);
  return hipGetLastError();
}

}  // namespace

// Called by the validated C entry point in gdn_capi.cpp.
hipError_t gdn_recurrent_step_launch(const gdn_tensor* q, const gdn_tensor* k, const gdn_tensor* v,
                                     const gdn_tensor* g, const gdn_tensor* beta, gdn_tensor* state,
                                     const gdn_tensor* idx, gdn_tensor* out, float scale, hipStream_t st) {
  RecurrentArgs a;
  a.q = q->data; a.k = k->data; a.v = v->data; a.g = g->data; a.beta = beta->data;
  a.state = reinterpret_cast<float*>(state->data); a.idx = idx->data; a.out = out->data;
  a.q_s0 = q->stride[0]; a.q_s1 = q->stride[1];
  a.k_s0 = k->stride[0]; a.k_s1 = k->stride[1];
  a.v_s0 = v->stride[0]; a.v_s1 = v->stride[1];
  a.g_s0 = g->stride[0]; a.g_s1 = g->stride[1];
  a.b_s0 = beta->stride[0]; a.b_s1 = beta->stride[1];
  a.o_s0 = out->stride[0]; a.o_s1 = out->stride[1];
  a.st_slot = state->stride[0]; a.st_head = state->stride[1];
  a.num_slots = state->shape[0];
  a.Hv = (int32_t)v->shape[1];
  a.r = (int32_t)(v->shape[1] / q->shape[1]);
  a.scale = scale;
  a.idx64 = idx->dtype == GDN_DTYPE_I64;
  a.g_dtype = g->dtype;
  a.b_dtype = beta->dtype;
  const int K = (int)q->shape[2], V = (int)v->shape[2];
  const int64_t nb = q->shape[0] * v->shape[1];
  if (nb == 0) return hipSuccess;
  switch (q->dtype) {  // out has v's dtype (validated by the caller)
    case GDN_DTYPE_BF16: return launch_dims<bf16_t>(a, K, V, nb, st);
    case GDN_DTYPE_F16: return launch_dims<f16_t>(a, K, V, nb, st);
    default: return launch_dims<float>(a, K, V, nb, st);
  }
}
