// Fused single-token decode step of one Gated DeltaNet layer: the causal
// conv1d update + SiLU of the packed q|k|v projections, the per-head L2 norm
// of q and k, the gate g = -exp(A_log) softplus(a + dt_bias) and
// beta = sigmoid(b), and the gated delta rule step, in one launch.
//
// It replaces the decode branch of GatedDeltaNet.forward in yuyifanbupt/myvllm
// (layers/linear_attention.py:89-90 gating, :95 causal_conv1d_update,
// :113-114 L2 norm, :119 recurrent_gated_delta_rule), which runs those pieces
// as separate launches (ops/causal_conv1d.py:276-470,
// ops/gated_delta_rule/fused_recurrent_gdn.py:6-166).
//
// One 1024-thread workgroup per (sequence, k-head) owns the k-head's q and k
// channels and the value channels of its NH = Hv / Hk v-heads, so every conv
// channel's state is advanced by exactly one workgroup.  The heads' fp32
// states (NH x 64 KiB) stream through with 16-byte non-temporal loads issued
// before the convolution, as in the plain decode step; the conv output, the
// normalised q and k, g and beta never leave the chip (fp32 throughout).
#include "gdn_common.h"

namespace {

struct FusedArgs {
  const void* x; const void* w; void* cs; const void* cidx;
  const void* ga; const void* gb; const void* A_log; const void* dt_bias;
  float* state; const void* sidx; void* out;
  int64_t x_s0, w_s0, w_s1, cs_s0, cs_s1, a_s0, a_s1, b_s0, b_s1, al_s0, dt_s0, o_s0, o_s1;
  int64_t st_slot, st_head;
  int64_t conv_slots, num_slots;
  int32_t Hk;
  int32_t w_dtype, cs_dtype, a_dtype, b_dtype, al_dtype, dt_dtype;
  float scale;
  bool cidx64, sidx64;
};

constexpr int kThreads = 1024;

GDN_DEVICE void store_scalar(void* p, int64_t off, int dtype, float v) {
  switch (dtype) {
    case GDN_DTYPE_BF16: reinterpret_cast<bf16_t*>(p)[off] = (bf16_t)v; break;
    case GDN_DTYPE_F16: reinterpret_cast<f16_t*>(p)[off] = (f16_t)v; break;
    default: reinterpret_cast<float*>(p)[off] = v; break;
  }
}

// torch.nn.functional.softplus with beta 1 and threshold 20
GDN_DEVICE float softplus_f32(float x) { return x > 20.f ? x : log1pf(__expf(x)); }

// One head fits two workgroups per CU (64 VGPRs).  With two or more heads the
// states alone take 32+ VGPRs per thread; forcing two workgroups per CU there
// spills freshly loaded state registers (measured 267 us against 203 us for
// batch 256 with two heads), so the register budget is left to the compiler.
template <typename TX, int W, int K, int V, int NH>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(NH <= 1 ? 8 : 4, 8)))
void gdn_decode_fused_kernel(FusedArgs a) {
  constexpr int CG = V / 4;             // float4 column groups per state row
  constexpr int RG = kThreads / CG;     // row groups
  constexpr int NI = K / RG;            // state rows per thread and head
  constexpr int WAVES = kThreads / 64;
  constexpr int NCH = 2 * K + NH * V;   // conv channels of one k-head group
  constexpr int QKW = 2 * K / 64;       // waves holding the q and k channels
  static_assert(NCH <= kThreads && K % 64 == 0 && kThreads % CG == 0 && K % RG == 0 && 64 % CG == 0 &&
                    CG * NH <= kThreads && NH <= 64,
                "shape");
  __shared__ float sq[K], sk[K], sv[NH][V];
  __shared__ float snorm[QKW];
  __shared__ float seg[NH];
  __shared__ float red[WAVES][NH][9][CG];
  __shared__ f32x4 sd[NH][CG];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t b = blockIdx.x / a.Hk;
  const int kh = (int)(blockIdx.x % a.Hk);
  const int h0 = kh * NH;
  const int c4 = tid % CG, r0 = tid / CG;
  const int64_t cslot = load_index(a.cidx, b, a.cidx64);
  const int64_t slot = load_index(a.sidx, b, a.sidx64);
  const bool conv_ok = cslot >= 0 && cslot < a.conv_slots;
  const bool ssm_ok = slot >= 0 && slot < a.num_slots;

  // Small inputs first: unconditional (clamped channel and slot indices) and
  // branch-free on their runtime dtypes, converted only once the state loads
  // are in flight (a load under a branch, or a conversion right after its
  // load, would wait for every earlier load).  Thread c < NCH owns conv
  // channel ch(c): q channels, then k channels, then the NH heads' v channels.
  const int c = tid < NCH ? tid : 0;
  const int64_t ch = c < K       ? (int64_t)kh * K + c
                     : c < 2 * K ? (int64_t)a.Hk * K + (int64_t)kh * K + (c - K)
                                 : 2 * (int64_t)a.Hk * K + (int64_t)h0 * V + (c - 2 * K);
  const int64_t cs_base = (conv_ok ? cslot : 0) * a.cs_s0 + ch;
  const TX xr = reinterpret_cast<const TX*>(a.x)[b * a.x_s0 + ch];
  ScalarRaw sraw[W - 1], wraw[W];
#pragma unroll
  for (int m = 0; m < W - 1; ++m) sraw[m] = load_scalar_raw(a.cs, cs_base + m * a.cs_s1, a.cs_dtype);
#pragma unroll
  for (int j = 0; j < W; ++j) wraw[j] = load_scalar_raw(a.w, ch * a.w_s0 + j * a.w_s1, a.w_dtype);

  // the heads' states (a padding sequence reads slot 0 and stores nothing):
  // the first head's now, the others once the conv inputs' registers are free
  float* S[NH];
  f32x4 s[NH][NI];
  auto load_state = [&](int n) {
    S[n] = a.state + (ssm_ok ? slot : 0) * a.st_slot + (h0 + n) * a.st_head;
#pragma unroll
    for (int i = 0; i < NI; ++i)
      s[n][i] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(S[n] + (int64_t)(r0 + RG * i) * V + 4 * c4));
  };
  load_state(0);

  // ---- conv update + SiLU, taps pre-scaled and accumulated newest first (as
  // causal_conv1d_step, so the conv output is the same number before rounding)
  float xt[W];
#pragma unroll
  for (int m = 0; m < W - 1; ++m) xt[m] = scalar_raw_f32(sraw[m], a.cs_dtype);
  xt[W - 1] = to_f32(xr);
  float acc = scalar_raw_f32(wraw[W - 1], a.w_dtype) * kNegLog2e * xt[W - 1];
#pragma unroll
  for (int m = 0; m < W - 1; ++m) acc = fmaf(scalar_raw_f32(wraw[m], a.w_dtype) * kNegLog2e, xt[m], acc);
  const float y = (conv_ok && tid < NCH) ? silu_from_scaled(acc) : 0.f;
  if (conv_ok && tid < NCH) {
#pragma unroll
    for (int m = 0; m < W - 1; ++m) store_scalar(a.cs, cs_base + m * a.cs_s1, a.cs_dtype, xt[m + 1]);
  }
#pragma unroll
  for (int n = 1; n < NH; ++n) load_state(n);
  // sums of squares of q and k (waves 0 .. QKW/2-1 hold q, the next QKW/2 hold k)
  float s2 = tid < 2 * K ? y * y : 0.f;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) s2 += __shfl_xor(s2, off, 64);
  if (lane == 0 && wave < QKW) snorm[wave] = s2;
  if (tid >= 2 * K && tid < NCH) sv[(tid - 2 * K) / V][(tid - 2 * K) % V] = y;
  __syncthreads();
  // L2 norm x rsqrt(sum x^2 + 1e-6); q also takes the attention scale
  if (tid < 2 * K) {
    const int w0 = tid < K ? 0 : QKW / 2;
    float ss = 0.f;
#pragma unroll
    for (int w = 0; w < QKW / 2; ++w) ss += snorm[w0 + w];
    const float rn = rsqrtf(ss + 1e-6f);
    if (tid < K) sq[tid] = y * rn * a.scale;
    else sk[tid - K] = y * rn;
  }
  __syncthreads();

  if (!ssm_ok) {  // padding sequence: zero output, state untouched
    for (int i = tid; i < NH * V; i += kThreads)
      reinterpret_cast<TX*>(a.out)[b * a.o_s0 + (h0 + i / V) * a.o_s1 + i % V] = from_f32<TX>(0.0f);
    return;
  }

  // ---- gated delta rule, S decayed first (fused_recurrent_gdn.py:96-99):
  //   kS = k^T S, qS = (scale q)^T S, d = beta (v - e^g kS),
  //   o = e^g qS + (scale q . k) d, S = e^g S + k d^T
  // partial reductions over this thread's rows, then over the wave's row
  // groups (lanes with equal c4 differ by CG), one head at a time
#pragma unroll
  for (int n = 0; n < NH; ++n) {
    float pk[4] = {0.f, 0.f, 0.f, 0.f}, pq[4] = {0.f, 0.f, 0.f, 0.f}, qk = 0.f;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const float kv = sk[r0 + RG * i];
      const float qv = sq[r0 + RG * i];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        pk[j] = fmaf(kv, s[n][i][j], pk[j]);
        pq[j] = fmaf(qv, s[n][i][j], pq[j]);
      }
      qk = fmaf(qv, kv, qk);
    }
#pragma unroll
    for (int off = CG; off < 64; off <<= 1) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        pk[j] += __shfl_xor(pk[j], off, 64);
        pq[j] += __shfl_xor(pq[j], off, 64);
      }
      qk += __shfl_xor(qk, off, 64);
    }
    if (lane < CG) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        red[wave][n][j][c4] = pk[j];
        red[wave][n][4 + j][c4] = pq[j];
      }
      red[wave][n][8][c4] = qk;
    }
  }
  __syncthreads();
  // CG x NH finisher threads form the head's gates (g = -exp(A_log)
  // softplus(a + dt_bias), beta = sigmoid(b); loaded only now, when the state
  // loads they would otherwise wait behind have landed), sum the waves'
  // partials and form d and the output
  if (tid < CG * NH) {
    const int n = tid / CG, cc = tid % CG;
    const int h = h0 + n;
    const float av = scalar_raw_f32(load_scalar_raw(a.ga, b * a.a_s0 + h * a.a_s1, a.a_dtype), a.a_dtype) +
                     scalar_raw_f32(load_scalar_raw(a.dt_bias, h * a.dt_s0, a.dt_dtype), a.dt_dtype);
    const float alog = scalar_raw_f32(load_scalar_raw(a.A_log, h * a.al_s0, a.al_dtype), a.al_dtype);
    const float bv = scalar_raw_f32(load_scalar_raw(a.gb, b * a.b_s0 + h * a.b_s1, a.b_dtype), a.b_dtype);
    const float eg = __expf(-__expf(alog) * softplus_f32(av));
    const float bn = 1.f / (1.f + __expf(-bv));
    if (cc == 0) seg[n] = eg;
    float kS[4] = {0.f, 0.f, 0.f, 0.f}, qS[4] = {0.f, 0.f, 0.f, 0.f}, qkn = 0.f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        kS[j] += red[w][n][j][cc];
        qS[j] += red[w][n][4 + j][cc];
      }
      qkn += red[w][n][8][cc];
    }
    f32x4 d;
#pragma unroll
    for (int j = 0; j < 4; ++j) d[j] = bn * (sv[n][4 * cc + j] - eg * kS[j]);
    sd[n][cc] = d;
    TX* o = reinterpret_cast<TX*>(a.out) + b * a.o_s0 + (h0 + n) * a.o_s1;
#pragma unroll
    for (int j = 0; j < 4; ++j) o[4 * cc + j] = from_f32<TX>(fmaf(eg, qS[j], qkn * d[j]));
  }
  __syncthreads();
#pragma unroll
  for (int n = 0; n < NH; ++n) {
    const float eg = seg[n];
    const f32x4 d = sd[n][c4];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const float kv = sk[r0 + RG * i];
      f32x4 t;
#pragma unroll
      for (int j = 0; j < 4; ++j) t[j] = fmaf(eg, s[n][i][j], kv * d[j]);
      __builtin_nontemporal_store(t, reinterpret_cast<f32x4*>(S[n] + (int64_t)(r0 + RG * i) * V + 4 * c4));
    }
  }
}

template <typename TX>
hipError_t launch_heads(const FusedArgs& a, int nh, int64_t nblocks, hipStream_t st) {
  switch (nh) {
    case 1: gdn_decode_fused_kernel<TX, 4, 128, 128, 1><<<dim3((unsigned)nblocks), dim3(kThreads), 0, st>>>(a); break;
    case 2: gdn_decode_fused_kernel<TX, 4, 128, 128, 2><<<dim3((unsigned)nblocks), dim3(kThreads), 0, st>>>(a); break;
    default: gdn_decode_fused_kernel<TX, 4, 128, 128, 4><<<dim3((unsigned)nblocks), dim3(kThreads), 0, st>>>(a); break;
  }
  return hipGetLastError();
}

}  // namespace

// Called by the validated C entry point in gdn_capi.cpp (conv width 4, head
// dims 128, Hv / Hk in {1, 2, 4}).
hipError_t gdn_decode_fused_launch(const gdn_tensor* x, const gdn_tensor* w, gdn_tensor* cs, const gdn_tensor* cidx,
                                   const gdn_tensor* ga, const gdn_tensor* gb, const gdn_tensor* A_log,
                                   const gdn_tensor* dt_bias, gdn_tensor* state, const gdn_tensor* sidx,
                                   gdn_tensor* out, int32_t Hk, float scale, hipStream_t st) {
  FusedArgs a;
  a.x = x->data; a.w = w->data; a.cs = cs->data; a.cidx = cidx->data;
  a.ga = ga->data; a.gb = gb->data; a.A_log = A_log->data; a.dt_bias = dt_bias->data;
  a.state = reinterpret_cast<float*>(state->data); a.sidx = sidx->data; a.out = out->data;
  a.x_s0 = x->stride[0];
  a.w_s0 = w->stride[0]; a.w_s1 = w->stride[1];
  a.cs_s0 = cs->stride[0]; a.cs_s1 = cs->stride[1];
  a.a_s0 = ga->stride[0]; a.a_s1 = ga->stride[1];
  a.b_s0 = gb->stride[0]; a.b_s1 = gb->stride[1];
  a.al_s0 = A_log->stride[0]; a.dt_s0 = dt_bias->stride[0];
  a.o_s0 = out->stride[0]; a.o_s1 = out->stride[1];
  a.st_slot = state->stride[0]; a.st_head = state->stride[1];
  a.conv_slots = cs->shape[0]; a.num_slots = state->shape[0];
  a.Hk = Hk;
  a.w_dtype = w->dtype; a.cs_dtype = cs->dtype; a.a_dtype = ga->dtype; a.b_dtype = gb->dtype;
  a.al_dtype = A_log->dtype; a.dt_dtype = dt_bias->dtype;
  a.scale = scale;
  a.cidx64 = cidx->dtype == GDN_DTYPE_I64;
  a.sidx64 = sidx->dtype == GDN_DTYPE_I64;
  const int nh = (int)(state->shape[1] / Hk);
  const int64_t nblocks = x->shape[0] * (int64_t)Hk;
  if (nblocks == 0) return hipSuccess;
  switch (x->dtype) {
    case GDN_DTYPE_BF16: return launch_heads<bf16_t>(a, nh, nblocks, st);
    case GDN_DTYPE_F16: return launch_heads<f16_t>(a, nh, nblocks, st);
    default: return launch_heads<float>(a, nh, nblocks, st);
  }
}
