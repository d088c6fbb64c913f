// Chunked gated-delta-rule prefill, fused into one kernel per (sequence, v-head).
//
// Replaces the six-kernel Triton pipeline of chunk_gated_delta_rule
// (ops/gated_delta_rule/gated_delta_rule.py:31-66 in yuyifanbupt/myvllm:
// cumsum.py, chunk_scaled_dot_kkt.py, solve_tril.py, wu.py, h.py, o.py), which
// round-trips A, w, u, the per-chunk states h and v_new through HBM.  Here a
// 256-thread workgroup walks the chunks of one sequence for one v-head and
// keeps everything on chip: the fp32 128x128 state lives in the registers of
// its 4 waves (wave w owns value columns [32w, 32w+32)), the chunk's K/Q/V
// tiles and the 64x64 chunk matrices live in LDS, and only q/k/v/g/beta are
// read and o written.
//
// Per chunk of L <= 64 tokens (gamma = in-chunk cumsum of g):
//   A  = strict_lower(beta_i k_i.k_j e^(gamma_i - gamma_j))    (kkt, bf16 MFMA)
//   P  = lower(q_i.k_j e^(gamma_i - gamma_j))                  (qk^T, bf16 MFMA)
//   T  = (I + A)^-1 diag(beta)                                 (fp32 block substitution)
//   R  = V - diag(e^gamma) K S                                 (split-bf16 MFMA)
//   V' = T R                       (= u - w S of the reference, split-bf16 MFMA)
//   O  = scale [diag(e^gamma) Q S + P V']                      (bf16 MFMA)
//   S  = e^gamma_L S + K^T diag(e^(gamma_L - gamma)) V'        (split-bf16 MFMA)
// The MFMAs run in fp16 (v_mfma_f32_32x32x16_f16, same rate as bf16): q and
// k are L2-normalised bf16 values, which fp16 holds exactly, and every fp32
// operand that feeds the carried state (S, R, the decayed V', and T) is split
// into fp16 hi + lo parts (22 mantissa bits).  Split operands are first
// scaled by a per-wave power of two (max |x| in [2^9, 2^10)) so fp16 can
// neither overflow nor flush them; the scale is undone on the fp32
// accumulator.  Products that only feed o use the hi part alone.
//
// MFMA: v_mfma_f32_32x32x16_f16.  Operand layouts (lane l, n = l % 32,
// g = l / 32): A[m][k] lane holds row n, 8 k; B[k][n] lane holds column n,
// 8 k; C lane holds column n, rows 8i + 4g + r (i, r < 4).  A C-layout tile
// whose rows are the contraction index is fed back as a B operand without
// any data movement by ordering the 16-wide k-step as
//   k = 16s + 8*(m / 4) + 4g + (m % 4),  m = 0..7 the operand slot,
// and every A operand is read from LDS in that same order.
#include "gdn_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int C = 64;      // chunk
constexpr int KD = 128;    // key head dim
constexpr int VD = 128;    // value head dim
constexpr int LDK = 152;   // bf16 row stride of the K/Q/V tiles (conflict-free b64 and transposed reads)
constexpr int LDT = 72;    // bf16 row stride of T_hi/T_lo/P
constexpr int LDA = 68;    // fp32 row stride of A/T

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

struct PrefillArgs {
  const bf16_t* q; const bf16_t* k; const bf16_t* v; const float* g; const void* beta;
  float* state; const void* idx; const void* cu; bf16_t* out;
  int64_t q_s0, q_s1, k_s0, k_s1, v_s0, v_s1, g_s0, g_s1, b_s0, b_s1, o_s0, o_s1;
  int64_t st_slot, st_head;
  int64_t T, nseq, num_slots;
  int32_t Hv, r;
  int32_t b_dtype;
  float scale;
  bool idx64, cu64;
};

struct Smem {
  f16_t k[C * LDK];   // chunk keys (fp16)
  f16_t q[C * LDK];   // chunk queries (fp16)
  bf16_t v[C * LDK];  // chunk values; also the staging buffer of the chunk's output
  float a[C * LDA];   // A, then T = (I + A)^-1 in place
  float m[3][16 * 17];
  f16_t thi[C * LDT];
  f16_t tlo[C * LDT];
  f16_t p[C * LDT];
  alignas(16) float gam[C];
  alignas(16) float eg[C];    // e^gamma
  alignas(16) float edec[C];  // e^(gamma_L - gamma), 0 past the chunk's last token
  alignas(16) float beta[C];
};

GDN_DEVICE f32x16 mfma(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

GDN_DEVICE f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int j = 0; j < 16; ++j) z[j] = 0.f;
  return z;
}

GDN_DEVICE f16x8 cat4(f16x4 lo, f16x4 hi) {
  return (f16x8){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// Operand fragment of a row-major bf16 LDS matrix M: lane holds
// M[r0 + n][k-step slots] -- an A operand (rows of M are the M dim) or a B
// operand of M^T (rows of M are the N dim).
GDN_DEVICE f16x8 frag_rows(const f16_t* M, int ld, int r0, int kbase, int lane) {
  const f16_t* p = M + (r0 + (lane & 31)) * ld + kbase + 4 * (lane >> 5);
  return cat4(*reinterpret_cast<const f16x4*>(p), *reinterpret_cast<const f16x4*>(p + 8));
}

// Operand fragment of the transpose of a row-major bf16 LDS matrix M: lane
// holds M[k-step slots][c0 + n], read with the LDS transpose unit
// (ds_read_b64_tr_b16: each 16-lane group reads a 4x16 block, lane i gets
// column i).
GDN_DEVICE f16x8 frag_cols(const f16_t* M, int ld, int c0, int kbase, int lane) {
  const int j = lane & 15, qd = lane >> 4;
  const f16_t* p = M + (kbase + 4 * (qd >> 1) + (j >> 2)) * ld + c0 + 16 * (qd & 1) + 4 * (j & 3);
  s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
  s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p + 8 * ld));
  return cat4(__builtin_bit_cast(f16x4, lo), __builtin_bit_cast(f16x4, hi));
}

// Rows 8i + 4g + (0..3) of the C-layout tile starting at row r0 hold token
// rows; fetch a per-row vector for them.
GDN_DEVICE f32x4 rows4(const float* vec, int r0, int i, int lane) {
  return *reinterpret_cast<const f32x4*>(vec + r0 + 8 * i + 4 * (lane >> 5));
}

// Power-of-two exponent e such that max|x| * 2^-e lies in [2^9, 2^10) over
// the wave's `nt` C tiles (0 when all are zero); the same on every lane.
GDN_DEVICE int wave_scale_exp(const f32x16* t, int nt) {
  float m = 0.f;
  for (int i = 0; i < nt; ++i)
#pragma unroll
    for (int j = 0; j < 16; ++j) m = fmaxf(m, fabsf(t[i][j]));
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  return m > 0.f ? __builtin_amdgcn_frexp_expf(m) - 10 : 0;
}

// hi/lo fp16 split of 8 fp32 values (registers 8h..8h+7 of a C tile) times sc
GDN_DEVICE void split8(const f32x16& c, int h, float sc, f16x8& hi, f16x8& lo) {
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    const float x = c[8 * h + m] * sc;
    const f16_t xh = (f16_t)x;
    hi[m] = xh;
    lo[m] = (f16_t)(x - (float)xh);
  }
}

GDN_DEVICE f16x8 round8(const f32x16& c, int h, float sc) {
  f16x8 r;
#pragma unroll
  for (int m = 0; m < 8; ++m) r[m] = (f16_t)(c[8 * h + m] * sc);
  return r;
}

__global__ __launch_bounds__(kThreads) void gdn_chunk_prefill_kernel(PrefillArgs a) {
  __shared__ Smem sm;
  __shared__ float gam_last;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int n = lane & 31;
  const int gq = lane >> 5;

  const int64_t seq = blockIdx.x / a.Hv;
  const int h = blockIdx.x % a.Hv;
  const int kh = h / a.r;
  int64_t s, e;
  seq_range(a.cu, a.cu64, seq, a.T, s, e);
  if (e <= s) return;
  const int64_t slot = load_index(a.idx, seq, a.idx64);
  if (slot < 0 || slot >= a.num_slots) {  // padding sequence: zero output rows, no state
    for (int64_t t = s + (tid >> 4); t < e; t += kThreads / 16) {
      bf16x8 z;
#pragma unroll
      for (int m = 0; m < 8; ++m) z[m] = (bf16_t)0.f;
      *reinterpret_cast<bf16x8*>(a.out + t * a.o_s0 + h * a.o_s1 + 8 * (tid & 15)) = z;
    }
    return;
  }

  // ---- state S (K x V fp32) in C layout: m-tile mt holds keys 32mt.., this wave's 32 columns
  float* Sg = a.state + slot * a.st_slot + h * a.st_head;
  const int col = 32 * wave + n;
  f32x16 S[4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int j = 0; j < 16; ++j) S[mt][j] = Sg[(32 * mt + 8 * (j >> 2) + 4 * gq + (j & 3)) * VD + col];

  const bf16_t* qg = a.q + kh * a.q_s1;
  const bf16_t* kg = a.k + kh * a.k_s1;
  const bf16_t* vg = a.v + h * a.v_s1;

  for (int64_t c0 = s; c0 < e; c0 += C) {
    const int L = (int)((e - c0) < C ? (e - c0) : C);
    __syncthreads();  // previous chunk is done with every LDS buffer

    // ---- load the chunk's K, Q (k-head, to fp16) and V (v-head) tiles; zero rows past L
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int vec = tid + u * kThreads;
      const int row = vec >> 4, cg = vec & 15;
      bf16x8 kv, qv, vv;
      if (row < L) {
        const int64_t t = c0 + row;
        kv = *reinterpret_cast<const bf16x8*>(kg + t * a.k_s0 + 8 * cg);
        qv = *reinterpret_cast<const bf16x8*>(qg + t * a.q_s0 + 8 * cg);
        vv = *reinterpret_cast<const bf16x8*>(vg + t * a.v_s0 + 8 * cg);
      } else {
#pragma unroll
        for (int m = 0; m < 8; ++m) { kv[m] = (bf16_t)0.f; qv[m] = (bf16_t)0.f; vv[m] = (bf16_t)0.f; }
      }
      f16x8 kh16, qh16;
#pragma unroll
      for (int m = 0; m < 8; ++m) { kh16[m] = (f16_t)(float)kv[m]; qh16[m] = (f16_t)(float)qv[m]; }
      *reinterpret_cast<f16x8*>(sm.k + row * LDK + 8 * cg) = kh16;
      *reinterpret_cast<f16x8*>(sm.q + row * LDK + 8 * cg) = qh16;
      *reinterpret_cast<bf16x8*>(sm.v + row * LDK + 8 * cg) = vv;
    }
    // ---- gamma = in-chunk cumsum of g; decay vectors (wave 0, one token per lane)
    if (wave == 0) {
      float gv = 0.f, bv = 0.f;
      if (lane < L) {
        gv = a.g[(c0 + lane) * a.g_s0 + h * a.g_s1];
        bv = load_scalar_f32(a.beta, (c0 + lane) * a.b_s0 + h * a.b_s1, a.b_dtype);
      }
      float gm = gv;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const float y = __shfl_up(gm, off, 64);
        if (lane >= off) gm += y;
      }
      const float gl = __shfl(gm, 63, 64);  // padded g is 0, so this is gamma at token L-1
      sm.gam[lane] = gm;
      sm.eg[lane] = __expf(gm);
      sm.edec[lane] = lane < L ? __expf(gl - gm) : 0.f;
      sm.beta[lane] = bv;
      if (lane == 0) gam_last = gl;
    }
    __syncthreads();

    // ---- A = strict_lower(beta_i G_ij e^(g_i - g_j)) and P = lower(QK^T e^(g_i - g_j))
    if (wave < 3) {
      const int mt = wave == 0 ? 0 : 1;
      const int nt = wave == 2 ? 1 : 0;
      f32x16 G = zero16(), Pq = zero16();
#pragma unroll
      for (int ks = 0; ks < KD / 16; ++ks) {
        const f16x8 bk = frag_rows(sm.k, LDK, 32 * nt, 16 * ks, lane);
        G = mfma(frag_rows(sm.k, LDK, 32 * mt, 16 * ks, lane), bk, G);
        Pq = mfma(frag_rows(sm.q, LDK, 32 * mt, 16 * ks, lane), bk, Pq);
      }
      const int j = 32 * nt + n;
      const float gj = sm.gam[j];
#pragma unroll
      for (int jj = 0; jj < 16; ++jj) {
        const int i = 32 * mt + 8 * (jj >> 2) + 4 * gq + (jj & 3);
        const float dec = i >= j ? __expf(sm.gam[i] - gj) : 0.f;
        sm.a[i * LDA + j] = i > j ? sm.beta[i] * G[jj] * dec : 0.f;
        sm.p[i * LDT + j] = (f16_t)(Pq[jj] * dec);
      }
    } else {  // upper 32x32 tiles are zero
      for (int x = lane; x < 32 * 32; x += 64) {
        const int i = x >> 5, j = 32 + (x & 31);
        sm.a[i * LDA + j] = 0.f;
        sm.p[i * LDT + j] = (f16_t)0.f;
      }
    }
    __syncthreads();

    // ---- T = (I + A)^-1: 16x16 diagonal blocks by forward substitution
    if (wave == 0) {
      const int b = lane >> 4, c = lane & 15;
      const float* Ab = sm.a + 16 * b * LDA + 16 * b;
      float x[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float acc = 0.f;
#pragma unroll
        for (int kk = 0; kk < i; ++kk) acc = fmaf(Ab[i * LDA + kk], x[kk], acc);
        x[i] = i == c ? 1.f : (i < c ? 0.f : -acc);
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) sm.a[(16 * b + i) * LDA + 16 * b + c] = x[i];
    }
    __syncthreads();
    // off-diagonal blocks, one block row at a time:
    //   T_ij = -T_ii sum_{k=j}^{i-1} A_ik T_kj
    {
      const int rr = tid >> 4, cc = tid & 15;
#pragma unroll
      for (int bi = 1; bi < 4; ++bi) {
        for (int bj = 0; bj < bi; ++bj) {
          float acc = 0.f;
          for (int bk = bj; bk < bi; ++bk) {
            const float* Ar = sm.a + (16 * bi + rr) * LDA + 16 * bk;
            const float* Tc = sm.a + (16 * bk) * LDA + 16 * bj + cc;
#pragma unroll
            for (int x = 0; x < 16; ++x) acc = fmaf(Ar[x], Tc[x * LDA], acc);
          }
          sm.m[bj][rr * 17 + cc] = acc;
        }
        __syncthreads();
        for (int bj = 0; bj < bi; ++bj) {
          const float* Tr = sm.a + (16 * bi + rr) * LDA + 16 * bi;
          float acc = 0.f;
#pragma unroll
          for (int x = 0; x < 16; ++x) acc = fmaf(Tr[x], sm.m[bj][x * 17 + cc], acc);
          sm.a[(16 * bi + rr) * LDA + 16 * bj + cc] = -acc;
        }
        __syncthreads();
      }
    }
    // ---- T' = T diag(beta) as hi/lo fp16
    for (int x = tid; x < C * C; x += kThreads) {
      const int i = x >> 6, j = x & 63;
      const float t = sm.a[i * LDA + j] * sm.beta[j];
      const f16_t th = (f16_t)t;
      sm.thi[i * LDT + j] = th;
      sm.tlo[i * LDT + j] = (f16_t)(t - (float)th);
    }
    __syncthreads();

    // ---- per-wave state products on this wave's 32 value columns
    const int es = wave_scale_exp(S, 4);
    const float ss = __builtin_amdgcn_ldexpf(1.f, -es);
    f16x8 shi[8], slo[8];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) split8(S[ks >> 1], ks & 1, ss, shi[ks], slo[ks]);

    f32x16 X[2], QS[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      X[mt] = zero16();
      QS[mt] = zero16();
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        const f16x8 ak = frag_rows(sm.k, LDK, 32 * mt, 16 * ks, lane);
        X[mt] = mfma(ak, shi[ks], X[mt]);
        X[mt] = mfma(ak, slo[ks], X[mt]);
        QS[mt] = mfma(frag_rows(sm.q, LDK, 32 * mt, 16 * ks, lane), shi[ks], QS[mt]);
      }
    }
    // R = V - diag(e^gamma) X  (X, QS are in units of 2^-es; V read transposed: rows are tokens)
    const float us = __builtin_amdgcn_ldexpf(1.f, es);
    f32x16 R[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f32x4 egv = rows4(sm.eg, 32 * mt, i, lane);
        const int j = lane & 15, qd = lane >> 4;
        const bf16_t* p = sm.v + (32 * mt + 8 * i + 4 * (qd >> 1) + (j >> 2)) * LDK + 32 * wave + 16 * (qd & 1) + 4 * (j & 3);
        const bf16x4 vv = __builtin_bit_cast(bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p));
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) R[mt][4 * i + rr] = (float)vv[rr] - egv[rr] * (X[mt][4 * i + rr] * us);
      }
    }
    const int er = wave_scale_exp(R, 2);
    const float rs = __builtin_amdgcn_ldexpf(1.f, -er);
    f16x8 rhi[4], rlo[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) split8(R[ks >> 1], ks & 1, rs, rhi[ks], rlo[ks]);
    // V' = T' R, in units of 2^-er (T' lower triangular: the first 32 rows need only k-steps 0, 1)
    f32x16 VN[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      VN[mt] = zero16();
#pragma unroll
      for (int ks = 0; ks < 2 * (mt + 1); ++ks) {
        const f16x8 ah = frag_rows(sm.thi, LDT, 32 * mt, 16 * ks, lane);
        const f16x8 al = frag_rows(sm.tlo, LDT, 32 * mt, 16 * ks, lane);
        VN[mt] = mfma(ah, rhi[ks], VN[mt]);
        VN[mt] = mfma(ah, rlo[ks], VN[mt]);
        VN[mt] = mfma(al, rhi[ks], VN[mt]);
      }
    }
    // O = scale (diag(e^gamma) Q S + P V'), staged as bf16 in this wave's columns of sm.v
    f16x8 vnb[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) vnb[ks] = round8(VN[ks >> 1], ks & 1, 1.f);
    const float ru = __builtin_amdgcn_ldexpf(1.f, er);
    const float qsu = __builtin_amdgcn_ldexpf(1.f, es - er);
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      f32x16 O;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f32x4 egv = rows4(sm.eg, 32 * mt, i, lane);
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) O[4 * i + rr] = egv[rr] * QS[mt][4 * i + rr] * qsu;
      }
#pragma unroll
      for (int ks = 0; ks < 2 * (mt + 1); ++ks) O = mfma(frag_rows(sm.p, LDT, 32 * mt, 16 * ks, lane), vnb[ks], O);
      const float osc = ru * a.scale;
#pragma unroll
      for (int jj = 0; jj < 16; ++jj) {
        const int row = 32 * mt + 8 * (jj >> 2) + 4 * gq + (jj & 3);
        sm.v[row * LDK + col] = (bf16_t)(O[jj] * osc);
      }
    }
    // S = e^gamma_L S + K^T diag(e^(gamma_L - gamma)) V'
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f32x4 dv = rows4(sm.edec, 32 * mt, i, lane);
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) VN[mt][4 * i + rr] *= dv[rr];
      }
    }
    const int ed = wave_scale_exp(VN, 2);
    const float ds = __builtin_amdgcn_ldexpf(1.f, -ed);
    f16x8 dhi[4], dlo[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) split8(VN[ks >> 1], ks & 1, ds, dhi[ks], dlo[ks]);
    // accumulate in units of 2^(er + ed): S_acc = S * 2^-(er+ed) + K^T Vd_scaled
    const float egl = __expf(gam_last);
    const float sin_ = egl * __builtin_amdgcn_ldexpf(1.f, -(er + ed));
    const float sout = __builtin_amdgcn_ldexpf(1.f, er + ed);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
      for (int j = 0; j < 16; ++j) S[mt][j] *= sin_;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const f16x8 akt = frag_cols(sm.k, LDK, 32 * mt, 16 * ks, lane);
        S[mt] = mfma(akt, dhi[ks], S[mt]);
        S[mt] = mfma(akt, dlo[ks], S[mt]);
      }
#pragma unroll
      for (int j = 0; j < 16; ++j) S[mt][j] *= sout;
    }
    __syncthreads();
    // ---- store the chunk's output rows
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int vec = tid + u * kThreads;
      const int row = vec >> 4, cg = vec & 15;
      if (row < L)
        *reinterpret_cast<bf16x8*>(a.out + (c0 + row) * a.o_s0 + h * a.o_s1 + 8 * cg) =
            *reinterpret_cast<const bf16x8*>(sm.v + row * LDK + 8 * cg);
    }
  }

  // ---- final state back to the slot
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int j = 0; j < 16; ++j) Sg[(32 * mt + 8 * (j >> 2) + 4 * gq + (j & 3)) * VD + col] = S[mt][j];
}

}  // namespace

hipError_t gdn_chunk_prefill_launch(const gdn_tensor* q, const gdn_tensor* k, const gdn_tensor* v,
                                    const gdn_tensor* g, const gdn_tensor* beta, gdn_tensor* state,
                                    const gdn_tensor* idx, const gdn_tensor* cu, gdn_tensor* out, float scale,
                                    hipStream_t st) {
  PrefillArgs a;
  a.q = reinterpret_cast<const bf16_t*>(q->data);
  a.k = reinterpret_cast<const bf16_t*>(k->data);
  a.v = reinterpret_cast<const bf16_t*>(v->data);
  a.g = reinterpret_cast<const float*>(g->data);
  a.beta = beta->data;
  a.state = reinterpret_cast<float*>(state->data);
  a.idx = idx->data;
  a.cu = cu->data;
  a.out = reinterpret_cast<bf16_t*>(out->data);
  a.q_s0 = q->stride[0]; a.q_s1 = q->stride[1];
  a.k_s0 = k->stride[0]; a.k_s1 = k->stride[1];
  a.v_s0 = v->stride[0]; a.v_s1 = v->stride[1];
  a.g_s0 = g->stride[0]; a.g_s1 = g->stride[1];
  a.b_s0 = beta->stride[0]; a.b_s1 = beta->stride[1];
  a.o_s0 = out->stride[0]; a.o_s1 = out->stride[1];
  a.st_slot = state->stride[0]; a.st_head = state->stride[1];
  a.T = q->shape[0];
  a.nseq = cu->shape[0] - 1;
  a.num_slots = state->shape[0];
  a.Hv = (int32_t)v->shape[1];
  a.r = (int32_t)(v->shape[1] / q->shape[1]);
  a.b_dtype = beta->dtype;
  a.scale = scale;
  a.idx64 = idx->dtype == GDN_DTYPE_I64;
  a.cu64 = cu->dtype == GDN_DTYPE_I64;
  const int64_t nblocks = a.nseq * a.Hv;
  if (nblocks == 0 || a.T == 0) return hipSuccess;
  gdn_chunk_prefill_kernel<<<dim3((unsigned)nblocks), dim3(kThreads), 0, st>>>(a);
  return hipGetLastError();
}
