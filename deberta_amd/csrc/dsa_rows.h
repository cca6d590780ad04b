// dsa_rows.h — the fused row kernels around the attention (gfx950): add +
// LayerNorm, bias + GELU and the RTD loss, forward and backward
// (include/dsa_block.h).  They are bound by HBM traffic: each reads its
// inputs once and writes its outputs once, in 8- or 16-byte vectors, with
// the statistics of a row in registers (one wave per row).  Column sums
// (parameter gradients) are taken per block of rows into a workspace and
// summed over the blocks in a fixed order by reduce_cols_kernel, so the
// results do not depend on scheduling.
//
// Element types of the row tensors are template parameters (float or
// bf16): a runtime type switch per load splits the code into many small
// blocks and costs registers and load batching.  Parameter vectors (bias,
// gamma, beta, w) keep a runtime type: they are read once per block.
#pragma once

#include "dsa_common.h"

namespace dsa {
namespace rows {

constexpr int kBF16 = 1;  // DSA_BF16 (DSA_F32 = 0)
constexpr int MAXC4 = 8;  // 4-element chunks a lane holds: C <= 64 * 4 * MAXC4 = 2048
// The row kernels are instantiated for NC chunks a lane, NC in {1, 2, 3, 4,
// 6, 8} and NC * 256 >= C, so that a row's registers stay at what C needs
// (C = 768: 3).
// Rows per block of the backward kernels: few rows a wave, so that a
// launch holds several waves per SIMD (the rows of a wave are serial); the
// column sums of the blocks are then many and short, summed by
// reduce_cols_kernel with sixteen waves a column group.
constexpr int LN_RB = 16;   // LayerNorm backward: 4 rows a wave
constexpr int GELU_RB = 8;   // GELU forward and backward: rows per thread
constexpr int RTD_RB = 8;   // RTD loss: 2 rows a wave

typedef float f4 __attribute__((ext_vector_type(4)));

// Typed row I/O: 4 elements at element offset i.
template <typename T>
struct Io;
template <>
struct Io<float> {
  static DSA_DEV f4 ld(const void* p, int64_t i) { return *reinterpret_cast<const f4*>(static_cast<const float*>(p) + i); }
  static DSA_DEV void st(void* p, int64_t i, f4 v) { *reinterpret_cast<f4*>(static_cast<float*>(p) + i) = v; }
};
template <>
struct Io<bf16> {
  static DSA_DEV f4 ld(const void* p, int64_t i) {
    const bf16x4 v = *reinterpret_cast<const bf16x4*>(static_cast<const bf16*>(p) + i);
    return f4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
  }
  static DSA_DEV void st(void* p, int64_t i, f4 v) {
    bf16x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = (bf16)v[e];
    *reinterpret_cast<bf16x4*>(static_cast<bf16*>(p) + i) = o;
  }
};

// Parameter vectors, runtime type.
DSA_DEV f4 ld4(const void* p, int64_t i, int dt) {
  return dt == kBF16 ? Io<bf16>::ld(p, i) : Io<float>::ld(p, i);
}
DSA_DEV float ld1(const void* p, int64_t i, int dt) {
  return dt == kBF16 ? (float)static_cast<const bf16*>(p)[i] : static_cast<const float*>(p)[i];
}
DSA_DEV void st1(void* p, int64_t i, float v, int dt) {
  if (dt == kBF16) static_cast<bf16*>(p)[i] = (bf16)v;
  else static_cast<float*>(p)[i] = v;
}

DSA_DEV float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

DSA_DEV f4 zero4() { return f4{0.f, 0.f, 0.f, 0.f}; }
DSA_DEV float hsum(f4 v) { return (v[0] + v[1]) + (v[2] + v[3]); }

// ---------------------------------------------------------------------------
// add + LayerNorm
struct LnParams {
  const void *x, *bias, *res, *gamma, *beta, *dy;
  void *y, *dz, *dgamma, *dbeta, *dbias;
  float *mean, *rstd, *part;
  int64_t xs, rs0, rs1, rpg, ys, dys, dzs, N;
  int C, pdt;
  float eps;
};

// the lane's parameter chunks (chunk k: columns 4 (lane + 64 k) .. + 3)
template <int NC>
DSA_DEV void ld_param(const void* p, int lane, int C4, int dt, f4 (&v)[NC]) {
#pragma unroll
  for (int k = 0; k < NC; ++k) v[k] = (p && lane + 64 * k < C4) ? ld4(p, 4 * (lane + 64 * k), dt) : zero4();
}

// z = x + bias + res for the lane's chunks of row r
template <int NC, typename TX, typename TR>
DSA_DEV void ln_load_z(const LnParams& p, int64_t r, int lane, const f4 (&bias)[NC], f4 (&z)[NC]) {
  const int C4 = p.C / 4;
  const int64_t rg = p.res ? r / p.rpg : 0, rsub = p.res ? r % p.rpg : 0;
  const int64_t rrow = rg * p.rs0 + rsub * p.rs1;
#pragma unroll
  for (int k = 0; k < NC; ++k) {
    const int c4 = lane + 64 * k;
    z[k] = zero4();
    if (c4 < C4) {
      z[k] = Io<TX>::ld(p.x, r * p.xs + 4 * c4) + bias[k];
      if (p.res) z[k] += Io<TR>::ld(p.res, rrow + 4 * c4);
    }
  }
}

// one wave per row
template <int NC, typename TX, typename TR, typename TY>
__global__ __launch_bounds__(256) void ln_fwd_kernel(LnParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= p.N) return;
  const int C4 = p.C / 4;
  f4 bias[NC], z[NC];
  ld_param<NC>(p.bias, lane, C4, p.pdt, bias);
  ln_load_z<NC, TX, TR>(p, r, lane, bias, z);
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < NC; ++k) s += hsum(z[k]);
  const float mean = wave_sum(s) / (float)p.C;
  float q = 0.f;
#pragma unroll
  for (int k = 0; k < NC; ++k)
    if (lane + 64 * k < C4) {
      const f4 d = z[k] - mean;
      q += hsum(d * d);
    }
  const float rstd = 1.0f / sqrtf(wave_sum(q) / (float)p.C + p.eps);
#pragma unroll
  for (int k = 0; k < NC; ++k) {
    const int c4 = lane + 64 * k;
    if (c4 < C4) {
      const f4 gm = ld4(p.gamma, 4 * c4, p.pdt), bt = ld4(p.beta, 4 * c4, p.pdt);
      Io<TY>::st(p.y, r * p.ys + 4 * c4, (z[k] - mean) * rstd * gm + bt);
    }
  }
  if (lane == 0) {
    p.mean[r] = mean;
    p.rstd[r] = rstd;
  }
}

// Rows [LN_RB * blockIdx.x, + LN_RB), LN_RB / 4 a wave.  dz = rstd * (g -
// mean(g) - xhat * mean(g * xhat)) with g = dy * gamma, written in x's
// type; the block's column sums of dy * xhat, dy and dz go to
// part[blockIdx.x][3][C].
template <int NC, typename TX, typename TR, typename TDY>
__global__ __launch_bounds__(256) void ln_bwd_kernel(LnParams p) {
  __shared__ float red[3 * 64 * 4 * NC];  // 3 sums x C
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int C4 = p.C / 4;
  f4 bias[NC], gm[NC], sg[NC], sb[NC], sz[NC];
  ld_param<NC>(p.bias, lane, C4, p.pdt, bias);
  ld_param<NC>(p.gamma, lane, C4, p.pdt, gm);
#pragma unroll
  for (int k = 0; k < NC; ++k) sg[k] = sb[k] = sz[k] = zero4();
#pragma unroll 1
  for (int u = 0; u < LN_RB / 4; ++u) {
    const int64_t r = (int64_t)blockIdx.x * LN_RB + w * (LN_RB / 4) + u;
    if (r >= p.N) break;
    f4 z[NC], dy[NC];
    ln_load_z<NC, TX, TR>(p, r, lane, bias, z);
#pragma unroll
    for (int k = 0; k < NC; ++k) dy[k] = lane + 64 * k < C4 ? Io<TDY>::ld(p.dy, r * p.dys + 4 * (lane + 64 * k)) : zero4();
    const float mean = p.mean[r], rstd = p.rstd[r];
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int k = 0; k < NC; ++k) {
      z[k] = lane + 64 * k < C4 ? (z[k] - mean) * rstd : zero4();  // xhat
      const f4 gg = dy[k] * gm[k];
      s1 += hsum(gg);
      s2 += hsum(gg * z[k]);
      sg[k] += dy[k] * z[k];
      sb[k] += dy[k];
    }
    const float m1 = wave_sum(s1) / (float)p.C, m2 = wave_sum(s2) / (float)p.C;
#pragma unroll
    for (int k = 0; k < NC; ++k) {
      const int c4 = lane + 64 * k;
      const f4 d = (dy[k] * gm[k] - m1 - z[k] * m2) * rstd;
      if (c4 < C4) Io<TX>::st(p.dz, r * p.dzs + 4 * c4, d);
      sz[k] += d;
    }
  }
  // the four waves' sums, added in wave order
  for (int v = 0; v < 4; ++v) {
    if (w == v) {
#pragma unroll
      for (int k = 0; k < NC; ++k) {
        const int c4 = lane + 64 * k;
        if (c4 < C4) {
          f4* a = reinterpret_cast<f4*>(red + 4 * c4);
          f4* b = reinterpret_cast<f4*>(red + p.C + 4 * c4);
          f4* c = reinterpret_cast<f4*>(red + 2 * p.C + 4 * c4);
          if (v == 0) {
            *a = sg[k];
            *b = sb[k];
            *c = sz[k];
          } else {
            *a += sg[k];
            *b += sb[k];
            *c += sz[k];
          }
        }
      }
    }
    __syncthreads();
  }
  f4* out = reinterpret_cast<f4*>(p.part + (int64_t)blockIdx.x * 3 * p.C);
  const f4* in = reinterpret_cast<const f4*>(red);
  for (int i = threadIdx.x; i < 3 * C4; i += 256) out[i] = in[i];
}

// ---------------------------------------------------------------------------
// bias + GELU (erf form: 0.5 z (1 + erf(z / sqrt 2)))
struct GeluParams {
  const void *x, *bias, *dy;
  void *y, *dz, *dbias;
  float* part;
  int64_t xs, ys, dys, dzs, N;
  int C, pdt;
};

// The erf GELU from one rational-exponential approximation of the
// complementary error function, Abramowitz & Stegun 7.1.26 (|error of erf|
// <= 1.5e-7 on x >= 0):
//   erfc(x) = t (a1 + t (a2 + t (a3 + t (a4 + t a5)))) exp(-x^2),  t = 1 / (1 + p x)
// With x = |z| / sqrt 2:  h = Phi(-|z|) = erfc(x) / 2 (the halving folded
// into the a_i, p divided by sqrt 2) and e = exp(-z^2 / 2), so
//   gelu(z)  = z Phi(z) = max(z, 0) - |z| h
//   gelu'(z) = Phi(z) + z phi(z) = (z >= 0 ? 1 - h : h) + z e / sqrt(2 pi)
// and the forward and the backward share the exponential: about 12 VALU
// operations and two transcendentals (v_rcp_f32, v_exp_f32) a value, where
// the library erff takes about 40 (the forward was bound by them).
struct GeluTail {
  float h;  // Phi(-|z|)
  float e;  // exp(-z^2 / 2)
};
DSA_DEV GeluTail gelu_tail(float z) {
  constexpr float kP = 0.3275911f * 0.70710678118654752f;
  constexpr float kA1 = 0.5f * 0.254829592f, kA2 = 0.5f * -0.284496736f, kA3 = 0.5f * 1.421413741f,
                  kA4 = 0.5f * -1.453152027f, kA5 = 0.5f * 1.061405429f;
  const float t = __builtin_amdgcn_rcpf(__builtin_fmaf(kP, fabsf(z), 1.f));
  float poly = __builtin_fmaf(t, kA5, kA4);
  poly = __builtin_fmaf(t, poly, kA3);
  poly = __builtin_fmaf(t, poly, kA2);
  poly = __builtin_fmaf(t, poly, kA1);
  GeluTail r;
  r.e = __builtin_amdgcn_exp2f((z * z) * (-0.5f * kLog2e));
  r.h = (poly * t) * r.e;
  return r;
}
DSA_DEV float gelu(float z) { return __builtin_fmaf(-fabsf(z), gelu_tail(z).h, fmaxf(z, 0.f)); }
DSA_DEV float gelu_grad(float z) {
  const GeluTail g = gelu_tail(z);
  const float phi_pos = z >= 0.f ? 1.f - g.h : g.h;
  return __builtin_fmaf(z * 0.39894228040143268f, g.e, phi_pos);
}

// block (column block, row block): thread per 4 columns, rows [GELU_RB *
// blockIdx.y, + GELU_RB), four rows' loads issued together
template <typename TX, typename TY>
__global__ __launch_bounds__(256) void gelu_fwd_kernel(GeluParams p) {
  const int c4 = blockIdx.x * 256 + threadIdx.x;
  if (4 * c4 >= p.C) return;
  const int c = 4 * c4;
  const f4 bv = p.bias ? ld4(p.bias, c, p.pdt) : zero4();
  const int64_t r0 = (int64_t)blockIdx.y * GELU_RB;
  for (int u0 = 0; u0 < GELU_RB; u0 += 4) {
    f4 z[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) z[u] = Io<TX>::ld(p.x, min(r0 + u0 + u, p.N - 1) * p.xs + c) + bv;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t r = r0 + u0 + u;
      if (r < p.N) {
        f4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = gelu(z[u][e]);
        Io<TY>::st(p.y, r * p.ys + c, o);
      }
    }
  }
}

// block (column block, row block): thread per 4 columns, rows [GELU_RB *
// blockIdx.y, + GELU_RB); dz in x's type; the row block's dbias partial to
// part[y][C] when dbias is asked for
template <typename TX, typename TDY>
__global__ __launch_bounds__(256) void gelu_bwd_kernel(GeluParams p) {
  const int c4 = blockIdx.x * 256 + threadIdx.x;
  if (4 * c4 >= p.C) return;
  const int c = 4 * c4;
  const f4 bv = p.bias ? ld4(p.bias, c, p.pdt) : zero4();
  f4 acc = zero4();
  const int64_t r0 = (int64_t)blockIdx.y * GELU_RB;
  // four rows at a time, their loads issued together
  for (int u0 = 0; u0 < GELU_RB; u0 += 4) {
    f4 z[4], dy[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t r = min(r0 + u0 + u, p.N - 1);
      z[u] = Io<TX>::ld(p.x, r * p.xs + c) + bv;
      dy[u] = Io<TDY>::ld(p.dy, r * p.dys + c);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t r = r0 + u0 + u;
      if (r < p.N) {
        f4 d;
#pragma unroll
        for (int e = 0; e < 4; ++e) d[e] = dy[u][e] * gelu_grad(z[u][e]);
        Io<TX>::st(p.dz, r * p.dzs + c, d);
        acc += d;
      }
    }
  }
  if (p.dbias) *reinterpret_cast<f4*>(p.part + (int64_t)blockIdx.y * p.C + c) = acc;
}

// Eight consecutive elements of a row as two 4-element halves (one 16-byte
// access for bf16, two for fp32).
template <typename T>
struct Io8 {
  typedef T v8 __attribute__((ext_vector_type(8)));
  static DSA_DEV void ld(const void* p, int64_t i, f4& a, f4& b) {
    if constexpr (sizeof(T) == 2) {
      const v8 v = *reinterpret_cast<const v8*>(static_cast<const T*>(p) + i);
      a = f4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
      b = f4{(float)v[4], (float)v[5], (float)v[6], (float)v[7]};
    } else {
      a = Io<T>::ld(p, i);
      b = Io<T>::ld(p, i + 4);
    }
  }
  static DSA_DEV void st(void* p, int64_t i, const f4& a, const f4& b) {
    if constexpr (sizeof(T) == 2) {
      v8 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = (T)a[e], v[4 + e] = (T)b[e];
      *reinterpret_cast<v8*>(static_cast<T*>(p) + i) = v;
    } else {
      Io<T>::st(p, i, a);
      Io<T>::st(p, i + 4, b);
    }
  }
};

// bias + GELU on rows whose element offsets and stride are multiples of 8
// (x, y and the bias aligned to 8 elements, C a multiple of 8): block
// (1024-column slab, row block), thread per 8 columns, rows [GELU_RB *
// blockIdx.y, + GELU_RB) with all their loads issued before the first
// store.
template <typename TX, typename TY>
__global__ __launch_bounds__(128) void gelu8_fwd_kernel(GeluParams p) {
  const int c = (blockIdx.x * 128 + threadIdx.x) * 8;
  if (c >= p.C) return;
  const f4 b0 = p.bias ? ld4(p.bias, c, p.pdt) : zero4(), b1 = p.bias ? ld4(p.bias, c + 4, p.pdt) : zero4();
  const int64_t r0 = (int64_t)blockIdx.y * GELU_RB;
  constexpr int NB = GELU_RB < 8 ? GELU_RB : 8;  // rows whose loads are issued together
#pragma unroll
  for (int u0 = 0; u0 < GELU_RB; u0 += NB) {
    f4 za[NB], zb[NB];
#pragma unroll
    for (int u = 0; u < NB; ++u) Io8<TX>::ld(p.x, min(r0 + u0 + u, p.N - 1) * p.xs + c, za[u], zb[u]);
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const int64_t r = r0 + u0 + u;
      if (r < p.N) {
        f4 oa, ob;
#pragma unroll
        for (int e = 0; e < 4; ++e) oa[e] = gelu(za[u][e] + b0[e]), ob[e] = gelu(zb[u][e] + b1[e]);
        Io8<TY>::st(p.y, r * p.ys + c, oa, ob);
      }
    }
  }
}

// the backward of gelu8_fwd_kernel: dz = dy gelu'(x + bias) in x's type, and
// the row block's dbias partial (column sums of dz) to part[y][C] when
// dbias is asked for
template <typename TX, typename TDY>
__global__ __launch_bounds__(128) void gelu8_bwd_kernel(GeluParams p) {
  const int c = (blockIdx.x * 128 + threadIdx.x) * 8;
  if (c >= p.C) return;
  const f4 b0 = p.bias ? ld4(p.bias, c, p.pdt) : zero4(), b1 = p.bias ? ld4(p.bias, c + 4, p.pdt) : zero4();
  const int64_t r0 = (int64_t)blockIdx.y * GELU_RB;
  f4 acc0 = zero4(), acc1 = zero4();
  constexpr int NB = 4;  // rows whose loads (x and dy) are issued together
#pragma unroll
  for (int u0 = 0; u0 < GELU_RB; u0 += NB) {
    f4 za[NB], zb[NB], ga[NB], gb[NB];
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const int64_t r = min(r0 + u0 + u, p.N - 1);
      Io8<TX>::ld(p.x, r * p.xs + c, za[u], zb[u]);
      Io8<TDY>::ld(p.dy, r * p.dys + c, ga[u], gb[u]);
    }
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const int64_t r = r0 + u0 + u;
      if (r < p.N) {
        f4 da, db;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          da[e] = ga[u][e] * gelu_grad(za[u][e] + b0[e]);
          db[e] = gb[u][e] * gelu_grad(zb[u][e] + b1[e]);
        }
        Io8<TX>::st(p.dz, r * p.dzs + c, da, db);
        acc0 += da;
        acc1 += db;
      }
    }
  }
  if (p.dbias) {
    *reinterpret_cast<f4*>(p.part + (int64_t)blockIdx.y * p.C + c) = acc0;
    *reinterpret_cast<f4*>(p.part + (int64_t)blockIdx.y * p.C + c + 4) = acc1;
  }
}

// ---------------------------------------------------------------------------
// RTD classifier + BCE loss
struct RtdParams {
  const void *x, *w, *b;
  const float* labels;
  const uint8_t* active;
  float *logits, *loss, *denom, *part;
  const float* dloss;
  void *dx, *dw, *db;
  int64_t xs, dxs, N;
  int C, pdt;
};

// logits of rows [RTD_RB * blockIdx.x, + RTD_RB), RTD_RB / 4 a wave; the
// block's (sum active * BCE, sum active) to part[2 * blockIdx.x]
template <int NC, typename TX>
__global__ __launch_bounds__(256) void rtd_fwd_kernel(RtdParams p) {
  __shared__ float red[8];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int C4 = p.C / 4;
  const float bias = p.b ? ld1(p.b, 0, p.pdt) : 0.f;
  f4 wv[NC];
  ld_param<NC>(p.w, lane, C4, p.pdt, wv);
  float lsum = 0.f, asum = 0.f;
#pragma unroll 1
  for (int u = 0; u < RTD_RB / 4; ++u) {
    const int64_t r = (int64_t)blockIdx.x * RTD_RB + w * (RTD_RB / 4) + u;
    if (r >= p.N) break;
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < NC; ++k) {
      const int c4 = lane + 64 * k;
      if (c4 < C4) s += hsum(Io<TX>::ld(p.x, r * p.xs + 4 * c4) * wv[k]);
    }
    const float zl = wave_sum(s) + bias;
    if (lane == 0) {
      p.logits[r] = zl;
      const float a = p.active ? (p.active[r] ? 1.f : 0.f) : 1.f;
      // BCE with logits, the stable form max(z, 0) - z y + log(1 + exp(-|z|))
      const float bce = fmaxf(zl, 0.f) - zl * p.labels[r] + log1pf(__expf(-fabsf(zl)));
      lsum += a * bce;
      asum += a;
    }
  }
  if (lane == 0) {
    red[2 * w] = lsum;
    red[2 * w + 1] = asum;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    p.part[2 * blockIdx.x] = red[0] + red[2] + red[4] + red[6];
    p.part[2 * blockIdx.x + 1] = red[1] + red[3] + red[5] + red[7];
  }
}

// the loss from the blocks' sums (one wave: lane i sums blocks i, i + 64,
// ..., then a fixed butterfly over the lanes)
__global__ __launch_bounds__(64) void rtd_loss_kernel(RtdParams p, int nblk) {
  float l = 0.f, a = 0.f;
  for (int i = threadIdx.x; i < nblk; i += 64) {
    l += p.part[2 * i];
    a += p.part[2 * i + 1];
  }
  l = wave_sum(l);
  a = wave_sum(a);
  if (threadIdx.x != 0) return;
  const float d = fmaxf(a, 1.f);
  p.denom[0] = d;
  p.loss[0] = l / d;
}

// dz_r = dloss * active_r * (sigmoid(logit_r) - label_r) / denom; dx_r =
// dz_r w; the block's column sums of dz_r x_r (dw) and its sum of dz_r (db)
// to part[blockIdx.x][C + 1]
template <int NC, typename TX, typename TDX>
__global__ __launch_bounds__(256) void rtd_bwd_kernel(RtdParams p) {
  constexpr int SDB = 64 * 4 * NC;  // the four waves' db sums after the C column sums
  __shared__ float red[SDB + 4];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int C4 = p.C / 4;
  const float g0 = p.dloss[0] / p.denom[0];
  f4 wv[NC], sw[NC];
  ld_param<NC>(p.w, lane, C4, p.pdt, wv);
#pragma unroll
  for (int k = 0; k < NC; ++k) sw[k] = zero4();
  float sdb = 0.f;
#pragma unroll 1
  for (int u = 0; u < RTD_RB / 4; ++u) {
    const int64_t r = (int64_t)blockIdx.x * RTD_RB + w * (RTD_RB / 4) + u;
    if (r >= p.N) break;
    const float a = p.active ? (p.active[r] ? 1.f : 0.f) : 1.f;
    const float zl = p.logits[r];
    const float dz = g0 * a * (1.f / (1.f + __expf(-zl)) - p.labels[r]);
    sdb += dz;
#pragma unroll
    for (int k = 0; k < NC; ++k) {
      const int c4 = lane + 64 * k;
      if (c4 < C4) {
        Io<TDX>::st(p.dx, r * p.dxs + 4 * c4, wv[k] * dz);
        sw[k] += Io<TX>::ld(p.x, r * p.xs + 4 * c4) * dz;
      }
    }
  }
  for (int v = 0; v < 4; ++v) {
    if (w == v) {
#pragma unroll
      for (int k = 0; k < NC; ++k) {
        const int c4 = lane + 64 * k;
        if (c4 < C4) {
          f4* a = reinterpret_cast<f4*>(red + 4 * c4);
          *a = v == 0 ? sw[k] : *a + sw[k];
        }
      }
      if (lane == 0) red[SDB + v] = sdb;
    }
    __syncthreads();
  }
  float* out = p.part + (int64_t)blockIdx.x * (p.C + 1);
  for (int i = threadIdx.x; i < p.C; i += 256) out[i] = red[i];
  if (threadIdx.x == 0) out[p.C] = red[SDB] + red[SDB + 1] + red[SDB + 2] + red[SDB + 3];
}

// ---------------------------------------------------------------------------
// out_j[k] = sum over parts i of part[i * stride + off_j + k], for the nout
// outputs j (column sums of the blocks' partials).  A block of 16 waves
// takes 64 columns: wave q sums parts q, q + 16, q + 32, ... into eight
// independent sums (eight loads in flight), then the sixteen waves' sums
// are added in wave order, so the result does not depend on scheduling.
constexpr int RED_W = 16;  // waves of a reduce block
struct ReduceCols {
  const float* part;
  int64_t nparts, stride;
  int K;
  int nout;
  int64_t off[3];
  void* out[3];
  int dt;
};
__global__ __launch_bounds__(64 * RED_W) void reduce_cols_kernel(ReduceCols rc) {
  __shared__ float red[RED_W][64];
  const int lane = threadIdx.x & 63, q = threadIdx.x >> 6;
  const int k = blockIdx.x * 64 + lane;
  const int j = blockIdx.y;
  if (j >= rc.nout || !rc.out[j]) return;  // uniform over the block
  float s = 0.f;
  if (k < rc.K) {
    const float* base = rc.part + rc.off[j] + k;
    float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    int64_t i = q;
    for (; i + 7 * RED_W < rc.nparts; i += 8 * RED_W) {
#pragma unroll
      for (int u = 0; u < 8; ++u) a[u] += base[(i + RED_W * u) * rc.stride];
    }
    for (; i < rc.nparts; i += RED_W) a[0] += base[i * rc.stride];
    s = ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
  }
  red[q][lane] = s;
  __syncthreads();
  if (q == 0 && k < rc.K) {
    float t = red[0][lane];
#pragma unroll
    for (int v = 1; v < RED_W; ++v) t += red[v][lane];
    st1(rc.out[j], k, t, rc.dt);
  }
}

}  // namespace rows
}  // namespace dsa
