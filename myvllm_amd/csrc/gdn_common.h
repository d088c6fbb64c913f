// Shared device helpers for the gfx950 kernels of libgdn_hip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/gdn_hip.h"

typedef __bf16 bf16_t;
typedef _Float16 f16_t;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

#define GDN_DEVICE __device__ __forceinline__

// ---- scalar conversions -------------------------------------------------
GDN_DEVICE float to_f32(float x) { return x; }
GDN_DEVICE float to_f32(bf16_t x) { return (float)x; }
GDN_DEVICE float to_f32(f16_t x) { return (float)x; }

template <typename T> GDN_DEVICE T from_f32(float x);
template <> GDN_DEVICE float from_f32<float>(float x) { return x; }
template <> GDN_DEVICE bf16_t from_f32<bf16_t>(float x) { return (bf16_t)x; }  // RNE (v_cvt_pk_bf16_f32)
template <> GDN_DEVICE f16_t from_f32<f16_t>(float x) { return (f16_t)x; }

// ---- 8-wide vector load/store of any element type as fp32 -----------------
// p must be 16-byte aligned for 2-byte types and 32-byte aligned for fp32
// (the host checks pointer and stride alignment before launch).
template <typename T> struct Vec8;
template <> struct Vec8<bf16_t> {
  static GDN_DEVICE void load(const bf16_t* p, float* f) {
    bf16x8 v = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = (float)v[i];
  }
  static GDN_DEVICE void store(bf16_t* p, const float* f) {
    bf16x8 v;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (bf16_t)f[i];
    *reinterpret_cast<bf16x8*>(p) = v;
  }
};
template <> struct Vec8<f16_t> {
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  static GDN_DEVICE void load(const f16_t* p, float* f) {
    h8 v = *reinterpret_cast<const h8*>(p);
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = (float)v[i];
  }
  static GDN_DEVICE void store(f16_t* p, const float* f) {
    h8 v;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (f16_t)f[i];
    *reinterpret_cast<h8*>(p) = v;
  }
};
template <> struct Vec8<float> {
  static GDN_DEVICE void load(const float* p, float* f) {
    f32x4 a = *reinterpret_cast<const f32x4*>(p);
    f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) { f[i] = a[i]; f[4 + i] = b[i]; }
  }
  static GDN_DEVICE void store(float* p, const float* f) {
    f32x4 a, b;
#pragma unroll
    for (int i = 0; i < 4; ++i) { a[i] = f[i]; b[i] = f[4 + i]; }
    *reinterpret_cast<f32x4*>(p) = a;
    *reinterpret_cast<f32x4*>(p + 4) = b;
  }
};

// The same 8 elements written with non-temporal stores: for streamed outputs
// that no kernel of the same launch reads back (measured 9 % faster on the
// varlen conv, whose output is half its HBM traffic).
template <typename T> GDN_DEVICE void store8_nt(T* p, const float* f) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  if constexpr (sizeof(T) == 2) {
    T v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = from_f32<T>(f[i]);
    __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(v), reinterpret_cast<u32x4*>(p));
  } else {
    const f32x4 a = {f[0], f[1], f[2], f[3]}, b = {f[4], f[5], f[6], f[7]};
    __builtin_nontemporal_store(a, reinterpret_cast<f32x4*>(p));
    __builtin_nontemporal_store(b, reinterpret_cast<f32x4*>(p + 4));
  }
}

// 8 consecutive elements kept in their storage type (fewer registers than
// fp32 while a batch of rows is in flight); expand() widens to fp32.
template <typename T> struct Raw8;
template <> struct Raw8<bf16_t> {
  bf16x8 v;
  GDN_DEVICE void load(const bf16_t* p) { v = *reinterpret_cast<const bf16x8*>(p); }
  GDN_DEVICE void expand(float* f) const {
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = (float)v[i];
  }
};
template <> struct Raw8<f16_t> {
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  h8 v;
  GDN_DEVICE void load(const f16_t* p) { v = *reinterpret_cast<const h8*>(p); }
  GDN_DEVICE void expand(float* f) const {
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = (float)v[i];
  }
};
template <> struct Raw8<float> {
  f32x4 a, b;
  GDN_DEVICE void load(const float* p) {
    a = *reinterpret_cast<const f32x4*>(p);
    b = *reinterpret_cast<const f32x4*>(p + 4);
  }
  GDN_DEVICE void expand(float* f) const {
#pragma unroll
    for (int i = 0; i < 4; ++i) { f[i] = a[i]; f[4 + i] = b[i]; }
  }
};

// Scalar of a runtime-typed float tensor (used for per-row scalars like g, beta).
GDN_DEVICE float load_scalar_f32(const void* p, int64_t off, int dtype) {
  switch (dtype) {
    case GDN_DTYPE_BF16: return (float)reinterpret_cast<const bf16_t*>(p)[off];
    case GDN_DTYPE_F16: return (float)reinterpret_cast<const f16_t*>(p)[off];
    default: return reinterpret_cast<const float*>(p)[off];
  }
}

// An fp32 / bf16 / fp16 scalar as two raw 16-bit halves, loaded without a
// branch on the dtype (for 16-bit types both halves are the element), and
// its value.  Keeping the load unconditional and the conversion separate
// lets the caller convert only after its other loads are in flight: a load
// inside a branch, or a conversion right after the load, makes the wave wait
// for every earlier vector load (they complete in order).
struct ScalarRaw {
  uint32_t lo, hi;
};
GDN_DEVICE ScalarRaw load_scalar_raw(const void* p, int64_t off, int dtype) {
  const int shift = dtype == GDN_DTYPE_F32 ? 2 : 1;  // log2 of the element size
  const uint16_t* e = reinterpret_cast<const uint16_t*>(reinterpret_cast<const char*>(p) + (off << shift));
  const int second = shift - 1;  // 1 for fp32 (the high half), 0 otherwise
  ScalarRaw r;
  r.lo = e[0];
  r.hi = e[second];
  return r;
}
GDN_DEVICE float scalar_raw_f32(ScalarRaw r, int dtype) {
  if (dtype == GDN_DTYPE_BF16) return __builtin_bit_cast(float, r.lo << 16);
  if (dtype == GDN_DTYPE_F16) return (float)__builtin_bit_cast(f16_t, (uint16_t)r.lo);
  return __builtin_bit_cast(float, (r.hi << 16) | r.lo);
}

// ---- SiLU of a convolution with pre-scaled taps --------------------------
// With the taps held pre-multiplied by -log2(e), a convolution gives
// a = -log2(e) * acc directly, and
//   silu(acc) = acc / (1 + e^-acc) = a / (-log2(e) * (1 + 2^a)),
// one exp2, one fma, one reciprocal and one multiply per element.
constexpr float kNegLog2e = -1.4426950408889634f;
GDN_DEVICE float silu_from_scaled(float a) {
  return a * __builtin_amdgcn_rcpf(fmaf(__builtin_amdgcn_exp2f(a), kNegLog2e, kNegLog2e));
}

// ---- index tensors (int32 or int64) ----------------------------------------
GDN_DEVICE int64_t load_index(const void* p, int64_t i, bool is64) {
  return is64 ? reinterpret_cast<const int64_t*>(p)[i] : (int64_t)reinterpret_cast<const int32_t*>(p)[i];
}

// Sequence n of a packed batch, clamped to [0, T] and to a non-negative length.
GDN_DEVICE void seq_range(const void* cu, bool cu64, int64_t n, int64_t T, int64_t& s, int64_t& e) {
  int64_t a = load_index(cu, n, cu64);
  int64_t b = load_index(cu, n + 1, cu64);
  a = a < 0 ? 0 : (a > T ? T : a);
  b = b < a ? a : (b > T ? T : b);
  s = a;
  e = b;
}

// Rows of a packed (T, H, Dv) output that no sequence covers -- [0, cu[0])
// and [cu[N], T), clamped like seq_range -- are set to zero, as the
// reference's ops allocate their outputs zero-filled (torch.zeros_like).
// The work is shared by all workgroups of a launch (a grid-stride loop over
// 16-byte vectors of those rows); when the sequences cover [0, T), the usual
// case, each thread only reads cu[0] and cu[N].  Dv * ES must be a multiple of
// 16 and rows 16-byte aligned (checked on the host).  Not inlined: its
// 64-bit index arithmetic would otherwise shape the register allocation of
// the whole kernel that calls it first thing.
template <int ES>
__device__ __attribute__((noinline)) void zero_uncovered_rows(void* out, int64_t s0, int64_t s1, int64_t H, int64_t Dv, const void* cu,
                                    bool cu64, int64_t nseq, int64_t T, int64_t wg, int64_t nwg, int64_t tid,
                                    int64_t nthreads) {
  int64_t first = load_index(cu, 0, cu64), last = load_index(cu, nseq, cu64);
  first = first < 0 ? 0 : (first > T ? T : first);
  last = last < first ? first : (last > T ? T : last);
  const int64_t nrows = first + (T - last);
  if (nrows == 0) return;
  typedef uint32_t u32x4z __attribute__((ext_vector_type(4)));
  constexpr int64_t per = 16 / ES;  // elements per 16-byte vector
  const int64_t vph = Dv / per, vpr = H * vph;
  for (int64_t i = wg * nthreads + tid; i < nrows * vpr; i += nwg * nthreads) {
    const int64_t r = i / vpr, rem = i - r * vpr;
    const int64_t h = rem / vph, c = (rem - h * vph) * per;
    const int64_t t = r < first ? r : last + (r - first);
    *reinterpret_cast<u32x4z*>(reinterpret_cast<char*>(out) + (t * s0 + h * s1 + c) * ES) = u32x4z{0u, 0u, 0u, 0u};
  }
}

// The same as a kernel of its own, for kernels whose register allocation a
// call would disturb: launched just before them on their stream (256 threads
// per workgroup, any grid).
template <int ES>
__global__ __launch_bounds__(256) void zero_uncovered_rows_kernel(void* out, int64_t s0, int64_t s1, int64_t H,
                                                                  int64_t Dv, const void* cu, bool cu64,
                                                                  int64_t nseq, int64_t T) {
  zero_uncovered_rows<ES>(out, s0, s1, H, Dv, cu, cu64, nseq, T, blockIdx.x, gridDim.x, threadIdx.x, 256);
}


// Sum over the 16 lanes of a DPP row, on every lane of the row (quad swaps,
// then the half-row and row mirrors).
template <int CTRL>
GDN_DEVICE float dpp_f32(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
GDN_DEVICE float row16_sum(float x) {
  x += dpp_f32<0xB1>(x);   // quad_perm [1,0,3,2]
  x += dpp_f32<0x4E>(x);   // quad_perm [2,3,0,1]
  x += dpp_f32<0x141>(x);  // row_half_mirror
  x += dpp_f32<0x140>(x);  // row_mirror
  return x;
}

// Inclusive prefix sum over the 64 lanes of a wave (DPP row shifts, then the
// row broadcasts of the last lane of each row).
GDN_DEVICE int wave_inclusive_scan_i32(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, false);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false);  // row_bcast:15 into rows 1, 3
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false);  // row_bcast:31 into rows 2, 3
  return x;
}

// Block-wide lookup of the (sequence, tile) pair owning linear tile id
// `target`, where sequence n is cut into ceil(len_n / tile_len) tiles laid
// out sequence after sequence.  Every thread of the (256-thread) block must
// call it; all receive the same answer, seq = -1 when target is past the end.
// Tile counts are 32-bit (the host bounds T and the grid).  `lds` must hold
// at least 6 int32 values.
template <int NT>
GDN_DEVICE void find_seq_tile(const void* cu, bool cu64, int64_t nseq, int64_t T, int tile_len, int64_t target,
                              int64_t& seq, int64_t& tile, int32_t* lds) {
  static_assert(NT == 256, "find_seq_tile assumes 256 threads");
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  __syncthreads();  // a previous call's readers of lds[4], lds[5] are done
  if (tid == 0) { lds[4] = -1; lds[5] = 0; }
  int64_t running = 0;
  for (int64_t base = 0; base < nseq; base += NT) {
    const int64_t n = base + tid;
    int cnt = 0;
    if (n < nseq) {
      int64_t s, e;
      seq_range(cu, cu64, n, T, s, e);
      cnt = (int)((e - s + tile_len - 1) / tile_len);
    }
    const int incl = wave_inclusive_scan_i32(cnt);
    __syncthreads();  // lds[0..3] free from the previous round
    if (lane == 63) lds[wave] = incl;
    __syncthreads();
    int wave_off = 0, total = 0;
#pragma unroll
    for (int w = 0; w < NT / 64; ++w) {
      const int tw = lds[w];
      if (w < wave) wave_off += tw;
      total += tw;
    }
    const int64_t hi = running + wave_off + incl;
    const int64_t lo = hi - cnt;
    if (cnt > 0 && target >= lo && target < hi) {
      lds[4] = (int32_t)n;
      lds[5] = (int32_t)(target - lo);
    }
    running += total;
    __syncthreads();
    if (lds[4] >= 0 || target < running) break;
  }
  seq = lds[4];
  tile = lds[5];
}
