// dsa_bwd.h — backward preparation kernel (gfx950): Delta_i = dO_i . O_i.
//
// The backward of the fused attention (ATen autograd of
// deberta_v2_native.py:592-652 with the c2p/p2c gathers of :389-410) is
//   dP = dO V^T,  dS = P * (dP - Delta),  Delta_i = dO_i . O_i
//   dV = P^T dO
//   dQ = s dS K   + s sum_j dS_ij Kr[c(i-j)],   dKr[r] = s sum_{c(i-j)=r} dS_ij q_i
//   dK = s dS^T Q + s sum_i dS_ij Qr[p(i-j)],   dQr[r] = s sum_{p(i-j)=r} dS_ij k_j
// with s the softmax scale; masked keys and dead query rows have P = 0 and so
// dS = 0.  dsa_bwd_dq.h computes dQ and dKr, dsa_bwd_dkdv.h dK, dV and dQr.
#pragma once

#include "dsa_tiles.h"

namespace dsa {

// ===========================================================================
// prep: delta_i = dO_i . O_i, and the transposed relative tables
// ===========================================================================
template <typename T, int D>
__global__ __launch_bounds__(256) void dsa_bwd_delta_kernel(BwdParams bp) {
  // D / VEC lanes per row, one 16-byte load each, then a butterfly sum.
  constexpr int VEC = 16 / sizeof(T);
  constexpr int LPR = D / VEC;
  typedef T vecT __attribute__((ext_vector_type(VEC)));
  const FwdParams& p = bp.f;
  const int64_t n = (int64_t)p.B * p.H * p.Lq;
  const int64_t row = ((int64_t)blockIdx.x * 256 + threadIdx.x) / LPR;
  const int part = threadIdx.x % LPR;
  float acc = 0.f;
  if (row < n) {
    const int i = (int)(row % p.Lq);
    const int h = (int)((row / p.Lq) % p.H);
    const int b = (int)(row / ((int64_t)p.Lq * p.H));
    const T* o = (const T*)p.out + (int64_t)b * p.os[0] + (int64_t)i * p.os[1] + (int64_t)h * p.os[2];
    const T* d = (const T*)bp.dout + (int64_t)b * bp.dos[0] + (int64_t)i * bp.dos[1] + (int64_t)h * bp.dos[2];
    const vecT ov = *reinterpret_cast<const vecT*>(o + part * VEC);
    const vecT dv = *reinterpret_cast<const vecT*>(d + part * VEC);
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc += (float)ov[e] * (float)dv[e];
  }
#pragma unroll
  for (int m = LPR / 2; m >= 1; m >>= 1) acc += __shfl_xor(acc, m);
  if (row < n && part == 0) bp.delta[row] = acc;
}

}  // namespace dsa
