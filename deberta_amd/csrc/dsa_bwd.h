// dsa_bwd.h — backward of the fused disentangled attention (gfx950): the
// math, the workspace it runs through, and the preparation kernels.
//
// With s the softmax scale (ATen autograd of deberta_v2_native.py:592-652
// and of the c2p/p2c gathers of :389-410):
//   dP = dO V^T,  dS = P * (dP - Delta),  Delta_i = dO_i . O_i
//   dV = P^T dO
//   dQ = s dS K   + s sum_j dS_ij Kr[c(i-j)],   dKr[r] = s sum_{c(i-j)=r} dS_ij q_i
//   dK = s dS^T Q + s sum_i dS_ij Qr[p(i-j)],   dQr[r] = s sum_{p(i-j)=r} dS_ij k_j
// Masked keys and dead query rows have P = 0 and so dS = 0.
//
// Kernels, in launch order:
//   prep   dsa_bwd_prep_kernel, one launch of three parts: prep_delta (lse
//          and Delta per row), prep_gather (krgt, qrgt: the relative tables
//          gathered per offset d = i - j and transposed, so a run of
//          consecutive offsets of one head-dim column is contiguous — the A
//          operand of the offset-band products) and prep_segments (the
//          offset range of each table row)
//   dkdv   dsa_bwd_dkdv_kernel (dsa_bwd_dkdv.h): recomputes the scores and
//          the softmax per (b, h, 128-key tile), writes dK, dV and dS
//          (rows = queries; bf16 for bf16 inputs), the only (L x L) tensor
//          the backward passes between its kernels
//   dq     dsa_bwd_dq_kernel (dsa_bwd_dq.h): dQ from dS, K and krgt
//   fold   dsa_bwd_table_kernel + dsa_bwd_fold_kernel (dsa_bwd_table.h):
//          the table gradients per offset, from dS, Q and K, then summed
//          onto table rows
#pragma once

#include "dsa_order.h"

namespace dsa {

// rowinfo[b][h][i] = (lse_i * log2 e, dO_i . O_i) for i < LqP: D / VEC lanes
// per row, one 16-byte load each, then a butterfly sum.  Rows past Lq get
// (inf, 0); dead rows already have lse = inf.  Block blk of 256 threads.
template <typename T, int D>
DSA_DEV void prep_delta(const BwdParams& bp, int blk) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int LPR = D / VEC;
  typedef T vecT __attribute__((ext_vector_type(VEC)));
  const FwdParams& p = bp.f;
  const int64_t n = (int64_t)p.B * p.H * p.LqP;
  const int64_t row = ((int64_t)blk * 256 + threadIdx.x) / LPR;
  const int part = threadIdx.x % LPR;
  float acc = 0.f;
  int i = 0, h = 0, b = 0;
  if (row < n) {
    i = (int)(row % p.LqP);
    h = (int)((row / p.LqP) % p.H);
    b = (int)(row / ((int64_t)p.LqP * p.H));
    if (i < p.Lq) {
      const T* o = (const T*)p.out + (int64_t)b * p.os[0] + (int64_t)i * p.os[1] + (int64_t)h * p.os[2];
      const T* d = (const T*)bp.dout + (int64_t)b * bp.dos[0] + (int64_t)i * bp.dos[1] + (int64_t)h * bp.dos[2];
      const vecT ov = *reinterpret_cast<const vecT*>(o + part * VEC);
      const vecT dv = *reinterpret_cast<const vecT*>(d + part * VEC);
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc += (float)ov[e] * (float)dv[e];
      if (sizeof(T) == 2 && p.olo) {
        // O's rounding residual (the forward's p.olo, with out's strides)
        const T* lo = (const T*)((uintptr_t)o + ((uintptr_t)p.olo - (uintptr_t)p.out));
        const vecT lv = *reinterpret_cast<const vecT*>(lo + part * VEC);
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc += (float)lv[e] * (float)dv[e];
      }
    }
  }
#pragma unroll
  for (int m = LPR / 2; m >= 1; m >>= 1) acc += __shfl_xor(acc, m);
  if (row < n && part == 0) {
    const float lse2 = (i < p.Lq) ? p.lse[((int64_t)b * p.H + h) * p.Lq + i] * kLog2e : INFINITY;
    *reinterpret_cast<float2*>(bp.rowinfo + 2 * row) = make_float2(lse2, acc);
  }
}

// Table row of offset d (clamped into the relative-position table's range).
DSA_DEV int offset_row(const int32_t* rel, int d, int Lq, int Lk, int A, bool p2c) {
  d = min(max(d, -(Lk - 1)), Lq - 1);
  const int t = min(max(rel[d + Lk - 1], -A), A);
  return p2c ? p2c_row(t, A) : c2p_row(t, A);
}

// krgt[h][d][t] = Kr[h][c(t' - OFF)][d] with t' = t ^ (VEC - 1) (each
// aligned group of VEC = 16 / sizeof(T) offsets reversed: the dq kernel's
// operand order), qrgt[h][d][t] = Qr[h][p(t - OFF)][d], for t in [0, TGP).
// One thread per (table, h, group of VEC consecutive t, d), d fastest: the
// lanes of a wave read one table row (coalesced) per element, and each
// thread stores its VEC gathered elements in one 16-byte store.  Block blk
// of 256 threads.
template <typename T, int D>
DSA_DEV void prep_gather(const BwdParams& bp, int blk) {
  constexpr int VEC = 16 / sizeof(T);
  typedef T vecT __attribute__((ext_vector_type(VEC)));
  const FwdParams& p = bp.f;
  const int NG = bp.TGP / VEC;
  const int64_t per = (int64_t)p.H * D * NG;
  const int64_t idx = (int64_t)blk * 256 + threadIdx.x;
  if (idx >= 2 * per) return;
  const bool q = idx >= per;
  if (q ? !(p.flags & 2) : !(p.flags & 1)) return;
  const int64_t r = q ? idx - per : idx;
  const int d = (int)(r % D);
  const int t0 = (int)((r / D) % NG) * VEC;
  const int h = (int)(r / ((int64_t)NG * D));
  const T* src = q ? (const T*)p.qr + (int64_t)h * p.qrs[0] : (const T*)p.kr + (int64_t)h * p.krs[0];
  const int64_t rs = q ? p.qrs[1] : p.krs[1];
  vecT v;
#pragma unroll
  for (int e = 0; e < VEC; ++e) {
    const int t = t0 + (q ? e : (VEC - 1 - e));
    v[e] = src[(int64_t)offset_row(p.rel, t - bp.OFF, p.Lq, p.Lk, p.A, q) * rs + d];
  }
  T* dst = (T*)(q ? bp.qrgt : bp.krgt) + ((int64_t)h * D + d) * bp.TGP + t0;
  *reinterpret_cast<vecT*>(dst) = v;
}

// seg[t][0][r], seg[t][1][r]: the offsets [begin, end) whose table row is r
// (t = 0: c2p, whose row is non-decreasing in the offset; t = 1: p2c,
// non-increasing).  One thread per (table, offset d), plus one past the
// last offset: it starts the rows above the previous offset's row, up to
// its own, and ends the rows from the previous offset's row up to (not
// including) its own.  Block blk of 256 threads.
DSA_DEV void prep_segments(const BwdParams& bp, int blk) {
  const FwdParams& p = bp.f;
  const int R = 2 * p.A, n = p.Lq + p.Lk - 1, dmin = -(p.Lk - 1);
  const int64_t idx = (int64_t)blk * 256 + threadIdx.x;
  if (idx >= 2 * (int64_t)(n + 1)) return;
  const int t = (int)(idx / (n + 1)), u = (int)(idx % (n + 1));
  if (!(p.flags & (1 << t))) return;
  // rows counted so that they are non-decreasing in d
  auto rank = [&](int d) {
    const int x = offset_row(p.rel, d, p.Lq, p.Lk, p.A, t == 1);
    return t ? R - 1 - x : x;
  };
  const int cur = u < n ? rank(dmin + u) : R;
  const int prev = u > 0 ? rank(dmin + u - 1) : -1;
  int* beg = bp.rowseg + (2 * t) * R;
  int* end = beg + R;
  for (int q = prev + 1; q <= min(cur, R - 1); ++q) beg[t ? R - 1 - q : q] = dmin + u;
  for (int q = max(prev, 0); q < min(cur, R); ++q) end[t ? R - 1 - q : q] = dmin + u;
}

// cinfo[b][c] = (lo, hi, all, 0) for the 32-token chunk c of batch row b
// under a key-padding or segment mask: the range of its nonzero segment
// ids (lo > hi if none) and whether every token of the chunk is active
// (tokens past L are inactive).  One thread per chunk.
DSA_DEV void prep_chunks(const BwdParams& bp, int blk) {
  const FwdParams& p = bp.f;
  const int nch = p.LqP / 32;
  const int64_t idx = (int64_t)blk * 256 + threadIdx.x;
  if (idx >= (int64_t)p.B * nch) return;
  const int b = (int)(idx / nch), c = (int)(idx % nch);
  int lo = 0x7fffffff, hi = (int)0x80000000, all = 1;
  for (int u = 0; u < 32; ++u) {
    const int i = 32 * c + u;
    const int s = i < p.Lq ? seg_at(p, b, i) : 0;
    if (s != 0) {
      lo = min(lo, s);
      hi = max(hi, s);
    } else {
      all = 0;
    }
  }
  bp.cinfo[idx] = int4{lo, hi, all, 0};
}

// The preparation stage in one launch: blocks [0, nb_gather) gather the
// tables, the next nb_seg blocks find the row segments, the next nb_chunk
// blocks summarise the mask's chunks, the rest compute rowinfo.  The short
// blocks go first and run beside the rowinfo blocks.
// Zeroes the table kernel's block accumulators (gacc_floats floats, a
// multiple of 4): one 16-byte store a thread.
DSA_DEV void prep_zero(const BwdParams& bp, int64_t gacc_floats, int blk) {
  const int64_t i = ((int64_t)blk * 256 + threadIdx.x) * 4;
  if (i < gacc_floats) *reinterpret_cast<f32x4*>(bp.gpart + i) = zero4();
}

struct PrepBlocks {
  int order, order_ny, gather, seg, chunk, zero, delta;
  int64_t gacc_floats;
};
// Blocks: the launch orders' cost blocks (dsa_order.h; batch row fastest,
// then the tile group, then the job) first, then gather, segments, chunk
// summaries, zeroing and rowinfo.
template <typename T, int D>
__global__ __launch_bounds__(256) void dsa_bwd_prep_kernel(BwdParams bp, PrepBlocks nb, OrderParams2 op2) {
  if ((int)blockIdx.x < nb.order) {
    const int k = blockIdx.x, B = op2.f.B;
    order_cost_block(op2, k % B, (k / B) % nb.order_ny, k / (B * nb.order_ny));
    return;
  }
  const int blk = blockIdx.x - nb.order;
  if (blk < nb.gather) {
    prep_gather<T, D>(bp, blk);
  } else if (blk < nb.gather + nb.seg) {
    prep_segments(bp, blk - nb.gather);
  } else if (blk < nb.gather + nb.seg + nb.chunk) {
    prep_chunks(bp, blk - nb.gather - nb.seg);
  } else if (blk < nb.gather + nb.seg + nb.chunk + nb.zero) {
    prep_zero(bp, nb.gacc_floats, blk - nb.gather - nb.seg - nb.chunk);
  } else {
    prep_delta<T, D>(bp, blk - nb.gather - nb.seg - nb.chunk - nb.zero);
  }
}

}  // namespace dsa
