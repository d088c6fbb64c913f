// Fused recurrent gated-delta-rule decode step (one token per sequence).
//
// Replaces the Triton kernel _fused_recurrent_gdn
// (ops/gated_delta_rule/fused_recurrent_gdn.py:6-102 in yuyifanbupt/myvllm),
// which tiles the fp32 state as 128x8 slabs (32 contiguous bytes per row).
// Here one 1024-thread workgroup owns the whole K x V fp32 state of one
// (sequence, v-head): every thread streams V/4-wide rows with 16-byte loads
// (a wave reads 1 KiB contiguous per instruction), both reductions over K
// (k^T S and q^T S) are done in the same pass, and the updated state is
// written back in place, so the state crosses HBM exactly once each way
// (non-temporal loads and stores: nothing of it is reused by this launch).
// The kernel template takes NH heads per workgroup; the launcher uses one.
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
  int32_t kd, vd;  // head dims of the PAD instantiation (multiples of 8 up to its K, V)
  bool idx64;
};

// 16 waves, 4 state rows each: the shortest load-to-store span per workgroup
// (measured against 256 / 512 threads and two heads per workgroup).
constexpr int kThreads = 1024;

// PAD: head dims a.kd <= K, a.vd <= V (multiples of 8) run in the K x V
// instantiation: state rows past kd and column groups past vd are neither
// loaded (zero) nor stored, q/k/v past the dims read as zero, and output
// columns past vd are not written; the state's rows are vd floats long.
template <typename TIn, int K, int V, int NH, bool PAD = false>
__global__ __launch_bounds__(kThreads) void gdn_recurrent_step_kernel(RecurrentArgs a) {
  constexpr int CG = V / 4;           // float4 column groups per row
  constexpr int RG = kThreads / CG;   // row groups
  constexpr int NI = K / RG;          // rows per thread
  constexpr int WAVES = kThreads / 64;
  static_assert(kThreads % CG == 0 && K % RG == 0 && 64 % CG == 0, "shape");

  static_assert(CG * NH <= kThreads, "finishers");
  __shared__ float sq[NH][K], sk[NH][K], sv[NH][V];
  __shared__ float red[WAVES][NH][9][CG];
  __shared__ f32x4 sd[NH][CG];

  const int tid = threadIdx.x;
  const int hpb = a.Hv / NH;  // workgroups per sequence
  const int64_t b = blockIdx.x / hpb;
  const int h0 = (int)(blockIdx.x % hpb) * NH;
  const int c4 = tid % CG;
  const int r0 = tid / CG;

  const int64_t slot = load_index(a.idx, b, a.idx64);
  if (slot < 0 || slot >= a.num_slots) {  // padding sequence: zero output, state untouched
#pragma unroll
    for (int n = 0; n < NH; ++n)
      if (tid < (PAD ? a.vd : V)) reinterpret_cast<TIn*>(a.out)[b * a.o_s0 + (h0 + n) * a.o_s1 + tid] = from_f32<TIn>(0.0f);
    return;
  }

  // The small inputs are loaded first, unconditionally (clamped indices) and
  // without dtype branches, and converted only after the state loads are in
  // flight: a conversion right after its load, or a load inside a branch,
  // would wait for every earlier load (vector loads complete in order).
  const int kd = PAD ? a.kd : K, vd = PAD ? a.vd : V;
  const int kj = tid < kd ? tid : 0;
  const int vj = tid >= kThreads - V && tid - (kThreads - V) < vd ? tid - (kThreads - V) : 0;
  TIn qr[NH], kr[NH], vr[NH];
  ScalarRaw graw[NH], braw[NH];
#pragma unroll
  for (int n = 0; n < NH; ++n) {
    const int h = h0 + n, kh = h / a.r;
    qr[n] = reinterpret_cast<const TIn*>(a.q)[b * a.q_s0 + kh * a.q_s1 + kj];
    kr[n] = reinterpret_cast<const TIn*>(a.k)[b * a.k_s0 + kh * a.k_s1 + kj];
    vr[n] = reinterpret_cast<const TIn*>(a.v)[b * a.v_s0 + h * a.v_s1 + vj];
    graw[n] = load_scalar_raw(a.g, b * a.g_s0 + h * a.g_s1, a.g_dtype);
    braw[n] = load_scalar_raw(a.beta, b * a.b_s0 + h * a.b_s1, a.b_dtype);
  }

  float* S[NH];
  f32x4 s[NH][NI];
  const int ld = PAD ? a.vd : V;  // state row length
  const bool colin = !PAD || 4 * c4 < a.vd;
#pragma unroll
  for (int n = 0; n < NH; ++n) {
    S[n] = a.state + slot * a.st_slot + (h0 + n) * a.st_head;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int r = r0 + RG * i;
      const bool in = colin && (!PAD || r < a.kd);
      const f32x4 x = __builtin_nontemporal_load(
          reinterpret_cast<const f32x4*>(S[n] + (in ? (int64_t)r * ld + 4 * c4 : 0)));
      s[n][i] = in ? x : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }

  float g[NH], beta[NH];
#pragma unroll
  for (int n = 0; n < NH; ++n) {
    if (tid < K) {
      sq[n][tid] = tid < kd ? to_f32(qr[n]) * a.scale : 0.f;
      sk[n][tid] = tid < kd ? to_f32(kr[n]) : 0.f;
    }
    if (tid >= kThreads - V) sv[n][tid - (kThreads - V)] = tid - (kThreads - V) < vd ? to_f32(vr[n]) : 0.f;
    g[n] = scalar_raw_f32(graw[n], a.g_dtype);
    beta[n] = scalar_raw_f32(braw[n], a.b_dtype);
  }
  __syncthreads();

  // partial reductions over this thread's rows
  float pk[NH][4], pq[NH][4], qk[NH];
#pragma unroll
  for (int n = 0; n < NH; ++n) {
#pragma unroll
    for (int j = 0; j < 4; ++j) pk[n][j] = pq[n][j] = 0.f;
    qk[n] = 0.f;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const float kv = sk[n][r0 + RG * i];
      const float qv = sq[n][r0 + RG * i];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        pk[n][j] = fmaf(kv, s[n][i][j], pk[n][j]);
        pq[n][j] = fmaf(qv, s[n][i][j], pq[n][j]);
      }
      qk[n] = fmaf(qv, kv, qk[n]);
    }
  }
  // reduce over row groups inside the wave (lanes with equal c4 differ by CG)
#pragma unroll
  for (int off = CG; off < 64; off <<= 1) {
#pragma unroll
    for (int n = 0; n < NH; ++n) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        pk[n][j] += __shfl_xor(pk[n][j], off, 64);
        pq[n][j] += __shfl_xor(pq[n][j], off, 64);
      }
      qk[n] += __shfl_xor(qk[n], off, 64);
    }
  }
  const int wave = tid >> 6;
  if ((tid & 63) < CG) {
#pragma unroll
    for (int n = 0; n < NH; ++n) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        red[wave][n][j][c4] = pk[n][j];
        red[wave][n][4 + j][c4] = pq[n][j];
      }
      red[wave][n][8][c4] = qk[n];
    }
  }
  __syncthreads();

  // CG x NH finisher threads sum the waves' partials, form d and the output,
  // and hand d back through LDS (every thread reading all partials would
  // multiply the LDS traffic by the number of row groups).
  if (tid < CG * NH) {
    const int n = tid / CG, c = tid % CG;
    float kS[4] = {0.f, 0.f, 0.f, 0.f}, qS[4] = {0.f, 0.f, 0.f, 0.f}, qkn = 0.f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        kS[j] += red[w][n][j][c];
        qS[j] += red[w][n][4 + j][c];
      }
      qkn += red[w][n][8][c];
    }
    float gn = g[0], bn = beta[0];
#pragma unroll
    for (int m = 1; m < NH; ++m)
      if (n == m) {
        gn = g[m];
        bn = beta[m];
      }
    const float eg = __expf(gn);
    f32x4 d;
#pragma unroll
    for (int j = 0; j < 4; ++j) d[j] = bn * (sv[n][4 * c + j] - eg * kS[j]);
    sd[n][c] = d;
    TIn* o = reinterpret_cast<TIn*>(a.out) + b * a.o_s0 + (h0 + n) * a.o_s1;
    if (4 * c < vd) {
#pragma unroll
      for (int j = 0; j < 4; ++j) o[4 * c + j] = from_f32<TIn>(fmaf(eg, qS[j], qkn * d[j]));
    }
  }
  __syncthreads();

#pragma unroll
  for (int n = 0; n < NH; ++n) {
    const float eg = __expf(g[n]);
    const f32x4 d = sd[n][c4];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int r = r0 + RG * i;
      const float kv = sk[n][r];
      f32x4 t;
#pragma unroll
      for (int j = 0; j < 4; ++j) t[j] = fmaf(eg, s[n][i][j], kv * d[j]);
      if (colin && (!PAD || r < a.kd)) __builtin_nontemporal_store(t, reinterpret_cast<f32x4*>(S[n] + (int64_t)r * ld + 4 * c4));
    }
  }
}

template <typename TIn, int K, int V, bool PAD = false>
hipError_t launch_heads(const RecurrentArgs& a, int64_t nitems, hipStream_t st) {
  gdn_recurrent_step_kernel<TIn, K, V, 1, PAD><<<dim3((unsigned)nitems), dim3(kThreads), 0, st>>>(a);
  return hipGetLastError();
}

// 128 x 128, 64 x 64 and 256 x 256 have their own instantiations; any other
// head dims (multiples of 8) run zero-padded in the 128 x 128 one when both
// are at most 128, else in the 256 x 256 one (one row group per wave there:
// 64 lanes x 4 columns span a 256-wide row).
template <typename TIn>
hipError_t launch_dims(const RecurrentArgs& a, int K, int V, int64_t nitems, hipStream_t st) {
  if (K == 128 && V == 128) return launch_heads<TIn, 128, 128>(a, nitems, st);
  if (K == 64 && V == 64) return launch_heads<TIn, 64, 64>(a, nitems, st);
  if (K <= 128 && V <= 128) return launch_heads<TIn, 128, 128, true>(a, nitems, st);
  if (K == 256 && V == 256) return launch_heads<TIn, 256, 256>(a, nitems, st);
  return launch_heads<TIn, 256, 256, true>(a, nitems, st);
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
  a.kd = (int32_t)q->shape[2];
  a.vd = (int32_t)v->shape[2];
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
