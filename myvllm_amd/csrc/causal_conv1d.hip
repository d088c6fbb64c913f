// Depthwise causal conv1d + SiLU: varlen prefill with conv-state carry, and
// the single-token decode update.
//
// Replaces the Triton kernels _causal_conv1d_fwd_kernel and
// _causal_conv1d_update_kernel (ops/causal_conv1d.py:6-218, :276-431 in
// yuyifanbupt/myvllm).  Both are HBM-streaming kernels: each thread owns 8
// consecutive channels (one 16-byte bf16 vector) and walks tokens, keeping
// the W-1 previous inputs in registers, so x is read once (plus a W-1 row
// halo per 64-token tile) and y written once, fully coalesced.
//
// Prefill tiling: each sequence is cut into 64-token tiles; blockIdx.x is a
// linear tile id resolved to (sequence, tile) on the device, so no host sync
// is needed (the reference calls .tolist() on cu_seqlens, ops/causal_conv1d.py:230).
// Only a sequence's first tile reads its old conv state (a later tile's
// window starts >= 64 > W-1 tokens into the sequence), and that same tile
// writes the new state, so the read-before-write order on a slot is the
// program order of one thread.
#include "gdn_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kTile = 64;  // tokens per prefill tile (>= W - 1, see the state-ownership note)
constexpr int kCh = 8;     // channels per thread
constexpr int kBatch = 8;  // token rows loaded together

struct ConvArgs {
  const void* x; const void* w; void* state; const void* idx; const void* cu; void* out;
  int64_t x_s0, w_s0, w_s1, st_s0, st_s1, o_s0;
  int64_t T, D, nseq, num_slots;
  int64_t norm_ch;  // channels [0, norm_ch) are L2-normalised per 128-channel head (0: none)
  bool idx64, cu64;
};

// Taps are held pre-multiplied by -log2(e) (silu_from_scaled, gdn_common.h).
GDN_DEVICE void scale_taps(float (*wr)[kCh], int W) {
  for (int j = 0; j < W; ++j)
#pragma unroll
    for (int c = 0; c < kCh; ++c) wr[j][c] *= kNegLog2e;
}

// The taps of this thread's 8 channels.  A contiguous, 16-byte aligned
// (D, W) weight puts them in 8 W consecutive elements, read as 16-byte
// vectors; any other layout is read element by element.
template <typename TW, int W>
GDN_DEVICE void load_weights(const ConvArgs& a, int64_t d0, float (*wr)[kCh]) {
  const TW* w = reinterpret_cast<const TW*>(a.w);
  if (a.w_s1 == 1 && a.w_s0 == W && (reinterpret_cast<uintptr_t>(w) & 15) == 0) {
    constexpr int kPer = 16 / (int)sizeof(TW);  // elements per 16-byte vector
    constexpr int kVec = kCh * W / kPer;
    static_assert((kCh * W) % kPer == 0, "whole vectors");
    typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
    const u32x4v* p = reinterpret_cast<const u32x4v*>(w + d0 * W);
    TW e[kCh * W];
#pragma unroll
    for (int i = 0; i < kVec; ++i) {
      const u32x4v v = p[i];
      const TW* ev = reinterpret_cast<const TW*>(&v);
#pragma unroll
      for (int m = 0; m < kPer; ++m) e[i * kPer + m] = ev[m];
    }
#pragma unroll
    for (int c = 0; c < kCh; ++c)
#pragma unroll
      for (int j = 0; j < W; ++j) wr[j][c] = to_f32(e[c * W + j]);
  } else {
#pragma unroll
    for (int j = 0; j < W; ++j)
#pragma unroll
      for (int c = 0; c < kCh; ++c) wr[j][c] = to_f32(w[(d0 + c) * a.w_s0 + j * a.w_s1]);
  }
}

// One tile (up to kTile tokens of one sequence) for this thread's 8 channels.
template <typename TX, typename TS, int W>
GDN_DEVICE void conv_tile(const ConvArgs& a, int64_t seq, int64_t tile, int64_t d0, const float (*wr)[kCh]) {
  int64_t s, e;
  seq_range(a.cu, a.cu64, seq, a.T, s, e);
  const int64_t slot = load_index(a.idx, seq, a.idx64);
  const bool has_state = slot >= 0 && slot < a.num_slots;
  const int64_t t0 = s + tile * kTile;
  const int64_t t1 = t0 + kTile < e ? t0 + kTile : e;

  const TX* x = reinterpret_cast<const TX*>(a.x);
  TX* out = reinterpret_cast<TX*>(a.out);
  if (!has_state) {  // padding sequence: zero output, state untouched
    float z[kCh] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int64_t t = t0; t < t1; ++t) Vec8<TX>::store(out + t * a.o_s0 + d0, z);
    return;
  }

  // window[m] = input at position t - (W-1) + m for the next token t
  float win[W - 1][kCh];
  TS* st = reinterpret_cast<TS*>(a.state) + slot * a.st_s0 + d0;
#pragma unroll
  for (int m = 0; m < W - 1; ++m) {
    const int64_t p = t0 - (W - 1) + m;
    if (p >= s) {
      Vec8<TX>::load(x + p * a.x_s0 + d0, win[m]);
    } else {  // only the first tile of a sequence gets here: old state row p - s + W - 1
      Vec8<TS>::load(st + (p - s + W - 1) * a.st_s1, win[m]);
    }
  }

  // The tile's kTile token rows in batches of kBatch, the next batch's loads in
  // flight while the current one is computed (two statically named buffers).
  // The tile is unrolled completely, so the window rotates by register
  // renaming.  Rows past the sequence end are loaded from its last row and
  // computed like the others (only their stores are skipped): no branch and
  // no wait on the loads.  Rows are addressed from the tile's first row with
  // 32-bit offsets (kTile * stride fits; checked on the host).
  const TX* xt = x + t0 * a.x_s0 + d0;
  TX* ot = out + t0 * a.o_s0 + d0;
  const int nt = (int)(t1 - t0);  // valid rows of this tile, 1..kTile
  const uint32_t xs = (uint32_t)a.x_s0, os = (uint32_t)a.o_s0;
  Raw8<TX> xa[kBatch], xb[kBatch];
  auto load_batch = [&](int r0, Raw8<TX>* dst) {
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const uint32_t r = (uint32_t)(r0 + u < nt ? r0 + u : nt - 1);
      dst[u].load(reinterpret_cast<const TX*>(reinterpret_cast<const char*>(xt) + r * xs * (uint32_t)sizeof(TX)));
    }
  };
  auto run_batch = [&](int r0, const Raw8<TX>* raw) {
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      float xr[kCh], y[kCh];
      raw[u].expand(xr);
#pragma unroll
      for (int c = 0; c < kCh; ++c) {
        float acc = wr[W - 1][c] * xr[c];
#pragma unroll
        for (int m = 0; m < W - 1; ++m) acc = fmaf(wr[m][c], win[m][c], acc);
        y[c] = silu_from_scaled(acc);
      }
      if (a.norm_ch > 0) {
        // per-head L2 norm x rsqrt(sum x^2 + 1e-6) of the q and k channels
        // (layers/linear_attention.py:113-114): a head's 128 channels are the
        // 8 channels of 16 consecutive lanes, one DPP row
        float ss = 0.f;
#pragma unroll
        for (int c = 0; c < kCh; ++c) ss = fmaf(y[c], y[c], ss);
        ss = row16_sum(ss);
        const float sc = d0 < a.norm_ch ? rsqrtf(ss + 1e-6f) : 1.f;
#pragma unroll
        for (int c = 0; c < kCh; ++c) y[c] *= sc;
      }
      if (r0 + u < nt)
        store8_nt(reinterpret_cast<TX*>(reinterpret_cast<char*>(ot) + (uint32_t)(r0 + u) * os * (uint32_t)sizeof(TX)), y);
#pragma unroll
      for (int m = 0; m < W - 2; ++m)
#pragma unroll
        for (int c = 0; c < kCh; ++c) win[m][c] = win[m + 1][c];
#pragma unroll
      for (int c = 0; c < kCh; ++c) win[W - 2][c] = xr[c];
    }
  };
  static_assert(kTile % (2 * kBatch) == 0, "whole batch pairs");
  load_batch(0, xa);
#pragma unroll
  for (int r = 0; r < kTile; r += 2 * kBatch) {
    load_batch(r + kBatch, xb);
    run_batch(r, xa);
    if (r + 2 * kBatch < kTile) load_batch(r + 2 * kBatch, xa);
    run_batch(r + kBatch, xb);
  }

  if (tile == 0) {  // new state = last W-1 rows of [old state; x_seq]
#pragma unroll
    for (int r = 0; r < W - 1; ++r) {
      const int64_t p = e - (W - 1) + r;
      float row[kCh];
      if (p >= s) {
        Vec8<TX>::load(x + p * a.x_s0 + d0, row);
      } else {  // old row p - s + W - 1 > r: not yet overwritten (rows are written in increasing order)
        Vec8<TS>::load(st + (p - s + W - 1) * a.st_s1, row);
      }
      Vec8<TS>::store(st + r * a.st_s1, row);
    }
  }
}

// One workgroup per (tile, channel block); blockIdx.x is the linear tile id.
template <typename TX, typename TW, typename TS, int W>
__global__ __launch_bounds__(kThreads) void causal_conv1d_varlen_kernel(ConvArgs a) {
  __shared__ int32_t lds[8];
  // output rows no sequence covers are zero, as the reference allocates y
  // zero-filled (ops/causal_conv1d.py:241)
  zero_uncovered_rows<(int)sizeof(TX)>(a.out, a.o_s0, 0, 1, a.D, a.cu, a.cu64, a.nseq, a.T,
                                       (int64_t)blockIdx.x * gridDim.y + blockIdx.y, (int64_t)gridDim.x * gridDim.y,
                                       threadIdx.x, kThreads);
  const int64_t d0 = ((int64_t)blockIdx.y * kThreads + threadIdx.x) * kCh;
  const bool active = d0 < a.D;
  // the taps depend only on the channel block: their loads overlap the lookup
  float wr[W][kCh];
  if (active) {
    load_weights<TW, W>(a, d0, wr);
    scale_taps(wr, W);
  }
  int64_t seq, tile;
  find_seq_tile<kThreads>(a.cu, a.cu64, a.nseq, a.T, kTile, blockIdx.x, seq, tile, lds);
  if (seq < 0 || !active) return;
  conv_tile<TX, TS, W>(a, seq, tile, d0, wr);
}

template <typename TX, typename TW, typename TS, int W>
__global__ __launch_bounds__(kThreads) void causal_conv1d_step_kernel(ConvArgs a) {
  const int64_t b = blockIdx.x;
  const int64_t d0 = ((int64_t)blockIdx.y * kThreads + threadIdx.x) * kCh;
  if (d0 >= a.D) return;
  const int64_t slot = load_index(a.idx, b, a.idx64);
  TX* out = reinterpret_cast<TX*>(a.out) + b * a.o_s0 + d0;
  if (slot < 0 || slot >= a.num_slots) {
    float z[kCh] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    Vec8<TX>::store(out, z);
    return;
  }
  TS* st = reinterpret_cast<TS*>(a.state) + slot * a.st_s0 + d0;
  float xt[W][kCh];
#pragma unroll
  for (int m = 0; m < W - 1; ++m) Vec8<TS>::load(st + m * a.st_s1, xt[m]);
  Vec8<TX>::load(reinterpret_cast<const TX*>(a.x) + b * a.x_s0 + d0, xt[W - 1]);
  float wr[W][kCh];
  load_weights<TW, W>(a, d0, wr);
  scale_taps(wr, W);
  float y[kCh];
#pragma unroll
  for (int c = 0; c < kCh; ++c) {
    // same order as the prefill kernel (newest tap first), so a decode update
    // and a one-token prefill give identical bits
    float acc = wr[W - 1][c] * xt[W - 1][c];
#pragma unroll
    for (int m = 0; m < W - 1; ++m) acc = fmaf(wr[m][c], xt[m][c], acc);
    y[c] = silu_from_scaled(acc);
  }
  Vec8<TX>::store(out, y);
#pragma unroll
  for (int m = 0; m < W - 1; ++m) Vec8<TS>::store(st + m * a.st_s1, xt[m + 1]);
}

template <typename TX, typename TW, typename TS>
hipError_t launch_width(bool varlen, const ConvArgs& a, int W, dim3 grid, hipStream_t st) {
#define GDN_CONV_CASE(WW)                                                                          \
  case WW:                                                                                         \
    if (varlen)                                                                                    \
      causal_conv1d_varlen_kernel<TX, TW, TS, WW><<<grid, dim3(kThreads), 0, st>>>(a);             \
    else                                                                                           \
      causal_conv1d_step_kernel<TX, TW, TS, WW><<<grid, dim3(kThreads), 0, st>>>(a);               \
    break;
  switch (W) {
    GDN_CONV_CASE(2)
    GDN_CONV_CASE(3)
    GDN_CONV_CASE(4)
    GDN_CONV_CASE(5)
    GDN_CONV_CASE(6)
    default: return hipErrorInvalidValue;
  }
#undef GDN_CONV_CASE
  return hipGetLastError();
}

template <typename TX, typename TW>
hipError_t launch_state(bool varlen, const ConvArgs& a, int sdt, int W, dim3 grid, hipStream_t st) {
  // conv state is either fp32 or x's dtype (validated by the caller)
  if (sdt == GDN_DTYPE_F32) return launch_width<TX, TW, float>(varlen, a, W, grid, st);
  return launch_width<TX, TW, TX>(varlen, a, W, grid, st);
}

template <typename TX>
hipError_t launch_weight(bool varlen, const ConvArgs& a, int wdt, int sdt, int W, dim3 grid, hipStream_t st) {
  // weight is either x's dtype or fp32 (validated by the caller)
  if (wdt == GDN_DTYPE_F32) return launch_state<TX, float>(varlen, a, sdt, W, grid, st);
  return launch_state<TX, TX>(varlen, a, sdt, W, grid, st);
}

hipError_t launch_conv(bool varlen, const gdn_tensor* x, const gdn_tensor* w, gdn_tensor* cs,
                       const gdn_tensor* idx, const gdn_tensor* cu, gdn_tensor* out, int64_t norm_ch, hipStream_t st) {
  ConvArgs a;
  a.norm_ch = norm_ch;
  a.x = x->data; a.w = w->data; a.state = cs->data; a.idx = idx->data;
  a.cu = cu ? cu->data : nullptr; a.out = out->data;
  a.x_s0 = x->stride[0]; a.w_s0 = w->stride[0]; a.w_s1 = w->stride[1];
  a.st_s0 = cs->stride[0]; a.st_s1 = cs->stride[1]; a.o_s0 = out->stride[0];
  a.T = x->shape[0]; a.D = x->shape[1];
  a.nseq = cu ? cu->shape[0] - 1 : x->shape[0];
  a.num_slots = cs->shape[0];
  a.idx64 = idx->dtype == GDN_DTYPE_I64;
  a.cu64 = cu && cu->dtype == GDN_DTYPE_I64;
  const int W = (int)w->shape[1];
  const int64_t ch_blocks = (a.D / kCh + kThreads - 1) / kThreads;
  int64_t gx;
  if (varlen) {
    gx = (a.T + kTile - 1) / kTile + a.nseq;  // upper bound on the number of tiles
  } else {
    gx = a.T;
  }
  if (gx == 0 || ch_blocks == 0) return hipSuccess;
  dim3 grid((unsigned)gx, (unsigned)ch_blocks);
  switch (x->dtype) {
    case GDN_DTYPE_BF16: return launch_weight<bf16_t>(varlen, a, w->dtype, cs->dtype, W, grid, st);
    case GDN_DTYPE_F16: return launch_weight<f16_t>(varlen, a, w->dtype, cs->dtype, W, grid, st);
    default: return launch_weight<float>(varlen, a, w->dtype, cs->dtype, W, grid, st);
  }
}

}  // namespace

hipError_t causal_conv1d_varlen_launch(const gdn_tensor* x, const gdn_tensor* w, gdn_tensor* cs,
                                       const gdn_tensor* idx, const gdn_tensor* cu, gdn_tensor* out,
                                       int64_t norm_ch, hipStream_t st) {
  return launch_conv(true, x, w, cs, idx, cu, out, norm_ch, st);
}

hipError_t causal_conv1d_step_launch(const gdn_tensor* x, const gdn_tensor* w, gdn_tensor* cs,
                                     const gdn_tensor* idx, gdn_tensor* out, hipStream_t st) {
  return launch_conv(false, x, w, cs, idx, nullptr, out, 0, st);
}
