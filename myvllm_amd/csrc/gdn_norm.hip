// Gated RMSNorm of the GDN output, per v-head:
//   y = x rsqrt(mean x^2 + eps) w silu(gate)      (fp32 math, output in x's dtype)
// as RMSNormGated (layers/norm.py:44-58 of yuyifanbupt/myvllm) applies it to
// o and z at layers/linear_attention.py:121.  A row is one (token, head).
// Rows of 128 elements (the layer's v-heads) take the fast kernel: 16 lanes
// x 8 elements (16-byte accesses), the sum of squares over a DPP row; each
// 16-lane group takes kRowsPer rows with all their loads in flight at once.
// Any other row length N (the reference takes any normalized_shape and
// reduces over its last dim) runs one wave per row, elements strided over the
// lanes, with a weight of N values or one row of N per head.
//
// Also the layer's gates, g = -exp(A_log) softplus(a + dt_bias) and
// beta = sigmoid(b) (layers/linear_attention.py:89-90), in fp32, one launch.
#include "gdn_common.h"

namespace {

struct NormArgs {
  const void* x; const void* gate; const void* w; void* out;
  int64_t x_s0, x_s1, g_s0, g_s1, o_s0, o_s1;
  int64_t rows, H, N;
  int64_t w_sh;  // weight stride per head (0: one weight row shared by all heads)
  int32_t w_dtype;
  float eps;
};

constexpr int kThreads = 256;
constexpr int kRowsPer = 4;                          // rows per 16-lane group
constexpr int kRows = kThreads / 16 * kRowsPer;      // rows per workgroup

template <typename T>
__global__ __launch_bounds__(kThreads) void rms_norm_gated_kernel(NormArgs a) {
  const int c0 = 8 * (threadIdx.x & 15);
  const int64_t row0 = (int64_t)blockIdx.x * kRows + (threadIdx.x >> 4);
  float wc[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) wc[c] = load_scalar_f32(a.w, c0 + c, a.w_dtype);
  // rows past the end are read from the last row (whole 16-lane groups, so
  // DPP rows stay complete) and not stored
  Raw8<T> xr[kRowsPer], gr[kRowsPer];
#pragma unroll
  for (int u = 0; u < kRowsPer; ++u) {
    int64_t row = row0 + (int64_t)u * (kThreads / 16);
    row = row < a.rows ? row : a.rows - 1;
    const int64_t t = row / a.H, h = row % a.H;
    xr[u].load(reinterpret_cast<const T*>(a.x) + t * a.x_s0 + h * a.x_s1 + c0);
    gr[u].load(reinterpret_cast<const T*>(a.gate) + t * a.g_s0 + h * a.g_s1 + c0);
  }
#pragma unroll
  for (int u = 0; u < kRowsPer; ++u) {
    const int64_t row = row0 + (int64_t)u * (kThreads / 16);
    float x[8], g[8];
    xr[u].expand(x);
    gr[u].expand(g);
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < 8; ++c) ss = fmaf(x[c], x[c], ss);
    const float r = rsqrtf(row16_sum(ss) * (1.f / 128.f) + a.eps);
    float y[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const float silu = g[c] / (1.f + __expf(-g[c]));
      y[c] = x[c] * r * wc[c] * silu;
    }
    if (row < a.rows) {
      const int64_t t = row / a.H, h = row % a.H;
      Vec8<T>::store(reinterpret_cast<T*>(a.out) + t * a.o_s0 + h * a.o_s1 + c0, y);
    }
  }
}

// Any row length: one wave per row, four rows per workgroup; the row is read
// twice (the second pass hits the cache), the sum of squares reduced over the
// wave with lane shuffles.
template <typename T>
__global__ __launch_bounds__(kThreads) void rms_norm_gated_any_kernel(NormArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (row >= a.rows) return;  // (whole waves: the shuffles below see every lane of the wave)
  const int64_t t = row / a.H, h = row % a.H;
  const T* x = reinterpret_cast<const T*>(a.x) + t * a.x_s0 + h * a.x_s1;
  const T* gt = reinterpret_cast<const T*>(a.gate) + t * a.g_s0 + h * a.g_s1;
  T* out = reinterpret_cast<T*>(a.out) + t * a.o_s0 + h * a.o_s1;
  const int64_t w0 = h * a.w_sh;
  float ss = 0.f;
  for (int64_t c = lane; c < a.N; c += 64) {
    const float v = to_f32(x[c]);
    ss = fmaf(v, v, ss);
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 64);
  const float r = rsqrtf(ss / (float)a.N + a.eps);
  for (int64_t c = lane; c < a.N; c += 64) {
    const float g = to_f32(gt[c]);
    const float silu = g / (1.f + __expf(-g));
    out[c] = from_f32<T>(to_f32(x[c]) * r * load_scalar_f32(a.w, w0 + c, a.w_dtype) * silu);
  }
}

struct GateArgs {
  const void* ga; const void* gb; const void* A_log; const void* dt_bias;
  float* g; float* beta;
  int64_t a_s0, b_s0, g_s0, be_s0;
  int64_t T, H;
  int32_t a_dtype, b_dtype, al_dtype, dt_dtype;
};

// torch.nn.functional.softplus with beta 1 and threshold 20
GDN_DEVICE float softplus_f32(float x) { return x > 20.f ? x : log1pf(__expf(x)); }

__global__ __launch_bounds__(kThreads) void gdn_gating_kernel(GateArgs a) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= a.T * a.H) return;
  const int64_t t = i / a.H, h = i % a.H;
  const float av = load_scalar_f32(a.ga, t * a.a_s0 + h, a.a_dtype) + load_scalar_f32(a.dt_bias, h, a.dt_dtype);
  const float bv = load_scalar_f32(a.gb, t * a.b_s0 + h, a.b_dtype);
  a.g[t * a.g_s0 + h] = -__expf(load_scalar_f32(a.A_log, h, a.al_dtype)) * softplus_f32(av);
  a.beta[t * a.be_s0 + h] = 1.f / (1.f + __expf(-bv));
}

}  // namespace

// Called by the validated C entry point in gdn_capi.cpp.  fast: 128-element
// rows, one shared weight row, 16-byte aligned rows (checked there).
hipError_t gdn_rms_norm_gated_launch(const gdn_tensor* x, const gdn_tensor* gate, const gdn_tensor* w,
                                     gdn_tensor* out, float eps, bool fast, hipStream_t st) {
  NormArgs a;
  a.x = x->data; a.gate = gate->data; a.w = w->data; a.out = out->data;
  a.x_s0 = x->stride[0]; a.x_s1 = x->stride[1];
  a.g_s0 = gate->stride[0]; a.g_s1 = gate->stride[1];
  a.o_s0 = out->stride[0]; a.o_s1 = out->stride[1];
  a.rows = x->shape[0] * x->shape[1];
  a.H = x->shape[1];
  a.N = x->shape[2];
  a.w_sh = w->ndim == 2 ? w->stride[0] : 0;
  a.w_dtype = w->dtype;
  a.eps = eps;
  if (a.rows == 0 || a.N == 0) return hipSuccess;
  if (!fast) {
    const dim3 grid((unsigned)((a.rows + kThreads / 64 - 1) / (kThreads / 64)));
    switch (x->dtype) {
      case GDN_DTYPE_BF16: rms_norm_gated_any_kernel<bf16_t><<<grid, dim3(kThreads), 0, st>>>(a); break;
      case GDN_DTYPE_F16: rms_norm_gated_any_kernel<f16_t><<<grid, dim3(kThreads), 0, st>>>(a); break;
      default: rms_norm_gated_any_kernel<float><<<grid, dim3(kThreads), 0, st>>>(a); break;
    }
    return hipGetLastError();
  }
  const int64_t blocks = (a.rows + kRows - 1) / kRows;
  switch (x->dtype) {
    case GDN_DTYPE_BF16: rms_norm_gated_kernel<bf16_t><<<dim3((unsigned)blocks), dim3(kThreads), 0, st>>>(a); break;
    case GDN_DTYPE_F16: rms_norm_gated_kernel<f16_t><<<dim3((unsigned)blocks), dim3(kThreads), 0, st>>>(a); break;
    default: rms_norm_gated_kernel<float><<<dim3((unsigned)blocks), dim3(kThreads), 0, st>>>(a); break;
  }
  return hipGetLastError();
}

// Called by the validated C entry point in gdn_capi.cpp.
hipError_t gdn_gating_launch(const gdn_tensor* ga, const gdn_tensor* gb, const gdn_tensor* A_log,
                             const gdn_tensor* dt_bias, gdn_tensor* g, gdn_tensor* beta, hipStream_t st) {
  GateArgs a;
  a.ga = ga->data; a.gb = gb->data; a.A_log = A_log->data; a.dt_bias = dt_bias->data;
  a.g = reinterpret_cast<float*>(g->data); a.beta = reinterpret_cast<float*>(beta->data);
  a.a_s0 = ga->stride[0]; a.b_s0 = gb->stride[0]; a.g_s0 = g->stride[0]; a.be_s0 = beta->stride[0];
  a.T = ga->shape[0]; a.H = ga->shape[1];
  a.a_dtype = ga->dtype; a.b_dtype = gb->dtype; a.al_dtype = A_log->dtype; a.dt_dtype = dt_bias->dtype;
  const int64_t n = a.T * a.H;
  if (n == 0) return hipSuccess;
  gdn_gating_kernel<<<dim3((unsigned)((n + kThreads - 1) / kThreads)), dim3(kThreads), 0, st>>>(a);
  return hipGetLastError();
}
