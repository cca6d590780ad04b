// dsa_bwd_table.h — gradients of the projected relative tables (gfx950).
//
//   dKr[r] = s sum_{b,i,j: c(i-j)=r} dS_ij q_i,   dQr[r] = s sum_{b,i,j: p(i-j)=r} dS_ij k_j
//
// are computed per offset d = i - j first,
//   Gc[d] = sum_{b,i} dS(i, i-d) q_i,   Gp[d] = sum_{b,j} dS(j+d, j) k_j,
// and then summed onto table rows (dsa_bwd_fold_kernel): c(d) and p(d) are
// monotone in d, so the offsets of one row form a contiguous range
// (dsa_bwd_segments_kernel finds them).
//
// dsa_bwd_table_kernel: one workgroup = (128-offset block [d0, d0+128),
// head h, batch group).  For each batch and each chunk of 32 queries
// [i0, i0+32) it stages the region of dS (rows = queries) with rows i0..,
// keys j in [jb, jb + 160), jb = i0 - d0 - 128 — which holds every pair of
// the chunk with an offset in the block — with the 32 query rows and a ring
// of key rows.  Element (r, c) of the staged region X has offset
// d = d0 + 127 - (c - r - 1); with e = c - r - 1 (so d = d0 + 127 - e):
//   Gc^T[e] += sum_r  Q^T[i0 + r] X[r][r + 1 + e]
//   Gp^T[e] += sum_c  K^T[jb + c] X[c - 1 - e][c]
// Both B operands walk a diagonal of X (eight single-element LDS reads per
// fragment); zero rows around X cover the out-of-chunk part of the walk.
// A wave's two offset blocks share their A operands (the p2c one over 64
// staged columns, with diagonal elements outside the chunk read as zeros).
// Wave w accumulates e in [32w, 32w + 32) in registers and writes them once,
// to a per-(block, head, batch group) partial.
#pragma once

#include "dsa_bwd.h"

namespace dsa {

namespace tbcfg {
constexpr int NW = 4;
constexpr int DBW = 128;           // offsets per block
constexpr int JC = 32;             // queries per step
constexpr int XC = DBW + JC;       // staged columns
constexpr int XP = 32;             // zero rows above the staged rows
constexpr int XROWS = XP + JC + 32;  // and 32 below
constexpr int XCOLS = DBW + 48;    // columns a diagonal walk can touch
constexpr int QRING = 256;         // ring rows kept (power of two >= XC)
}  // namespace tbcfg

// Transposed LDS operand read (see tr_contig) from a ring of rows: logical
// row k lives at physical row (kbase + k) % QRING.
template <typename T>
DSA_DEV typename Mfma<T>::frag tr_contig_ring(const T* X, int str, int kbase, int k0, int m0, int g, int c16) {
  using namespace tbcfg;
  if constexpr (sizeof(T) == 2) {
    const int r0 = (kbase + k0 + 8 * g) & (QRING - 1);      // 4-aligned, so
    const int r1 = (kbase + k0 + 8 * g + 4) & (QRING - 1);  // rows never wrap
    return join8(tr4(X, str, r0, m0, c16), tr4(X, str, r1, m0, c16));
  } else {
    return tr4(X, str, (kbase + k0 + 4 * g) & (QRING - 1), m0, c16);
  }
}

// Rows [r0, r0 + n) of a [L, D] strided matrix into ring rows (zeros for rows
// outside [0, nvalid)).
template <typename T, int D>
DSA_DEV void load_ring_rows(T* ring, int str, const T* src, int64_t rs, int r0, int n, int nvalid, int tid) {
  using namespace tbcfg;
  constexpr int VEC = 16 / sizeof(T);
  constexpr int CPR = D / VEC;
  typedef T vecT __attribute__((ext_vector_type(VEC)));
  for (int c = tid; c < n * CPR; c += 256) {
    const int r = r0 + c / CPR, d0 = (c % CPR) * VEC;
    vecT x;
    if (r >= 0 && r < nvalid) {
      x = *reinterpret_cast<const vecT*>(src + (int64_t)r * rs + d0);
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) x[e] = (T)0.0f;
    }
    *reinterpret_cast<vecT*>(ring + (r & (QRING - 1)) * str + d0) = x;
  }
}

// Number of 32-query chunks of offset block dblk that hold pairs with an
// offset in the block, and the first of them: rows i >= d0 (a key j = i - d
// >= 0 exists) and i0 - d0 - 127 <= Lk - 1 (a key j < Lk exists).
DSA_DEV void block_chunks(int dblk, int LkP, int Lq, int Lk, int* istart, int* nch) {
  using namespace tbcfg;
  const int d0 = -LkP + DBW * dblk;  // a multiple of 128
  const int is = d0 > 0 ? d0 : 0;
  const int ie = min(Lq, Lk + d0 + DBW - 1);
  *istart = is;
  *nch = ie > is ? (ie - is + JC - 1) / JC : 0;
}

template <typename T, int D>
__global__ __launch_bounds__(256, 2) void dsa_bwd_table_kernel(BwdParams bp) {
  using namespace tbcfg;
  using M = Mfma<T>;
  typedef typename M::frag frag;
  constexpr int VEC = 16 / sizeof(T);
  typedef T vecT __attribute__((ext_vector_type(VEC)));
  constexpr int ND = D / 16;
  constexpr int FE = M::FRAG_ELEMS;
  constexpr int KSTR = D + Pad<T>::v;
  // Row stride of X chosen for few LDS bank conflicts in its diagonal walks
  // (178: two-way at most; rows are then only 4-byte aligned).
  constexpr int XSTR = sizeof(T) == 2 ? 178 : XCOLS + Pad<T>::v;
  constexpr int RSTR = KSTR;
  constexpr int GP_STEPS = 64 / M::KSTEP;  // k steps over the 64 staged columns a wave's two blocks read
  constexpr int GC_STEPS = JC / M::KSTEP;
  constexpr int XV = JC * XC / VEC;   // 16-byte chunks of the staged region
  constexpr int RV = JC * D / VEC;    // 16-byte chunks of 32 query (or key) rows
  constexpr int XCH = (XV + 255) / 256, RCH = (RV + 255) / 256;
  const FwdParams& p = bp.f;

  __shared__ __align__(16) T Xs[XROWS * XSTR];
  __shared__ __align__(16) T Qc[JC * KSTR];          // the chunk's query rows
  __shared__ __align__(16) T Kring[QRING * RSTR];    // key rows of the staged columns

  const int tid = threadIdx.x;
  const int w = tid >> 6, g = (tid & 63) >> 4, c16 = tid & 15;
  // Work order: blockIdx.x enumerates (offset block, head, batch group) with
  // the offset blocks that have the most chunks first, so the shortest
  // workgroups fill in at the end of the launch.  (Grouping a (head, batch
  // group)'s offset blocks on one XCD instead measured slower: the long
  // blocks then finish last.)
  const int per_blk = p.H * bp.NBG;
  const int rank = blockIdx.x / per_blk, rem = blockIdx.x % per_blk;
  const int h = rem / bp.NBG, bg = rem % bp.NBG;
  const int mid = (bp.NDB - 1) / 2;   // central blocks hold the most pairs
  const int dblk = (rank & 1) ? mid + 1 + (rank >> 1) : mid - (rank >> 1);
  const int d0 = -bp.f.LkP + DBW * dblk;
  const bool c2p = (p.flags & 1) != 0, p2c = (p.flags & 2) != 0;
  const int b_lo = bg * bp.BPG, b_hi = min(p.B, b_lo + bp.BPG);
  int istart, nch;
  block_chunks(dblk, bp.f.LkP, p.Lq, p.Lk, &istart, &nch);
  const int nsteps = (b_hi > b_lo) ? (b_hi - b_lo) * nch : 0;

  // zero rows around the staged region (never overwritten), and a finite ring
  {
    vecT z;
#pragma unroll
    for (int e = 0; e < VEC; ++e) z[e] = (T)0.0f;
    static_assert(XROWS * XSTR % VEC == 0 && QRING * RSTR % VEC == 0, "whole 16-byte chunks");
    for (int c = tid; c < XROWS * XSTR / VEC; c += 256) reinterpret_cast<vecT*>(Xs)[c] = z;
    for (int c = tid; c < QRING * RSTR / VEC; c += 256) reinterpret_cast<vecT*>(Kring)[c] = z;
  }

  f32x4 gc[2][ND], gp[2][ND];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int db = 0; db < ND; ++db) gc[t][db] = gp[t][db] = zero4();

  // Registers holding the next step's global data.
  vecT xr[XCH], qr[RCH], kr[RCH];
  auto step_coords = [&](int st, int& b, int& i0) {
    b = b_lo + st / nch;
    i0 = istart + (st % nch) * JC;
  };
  auto fetch = [&](int st) {
    int b, i0;
    step_coords(st, b, i0);
    const int jb = i0 - d0 - DBW;  // key of staged column 0 (a multiple of 32)
    const T* dsb = (const T*)bp.ds + (int64_t)(b * p.H + h) * bp.f.LqP * bp.f.LkP;
#pragma unroll
    for (int k = 0; k < XCH; ++k) {
      const int c = tid + 256 * k;
      const int r = c / (XC / VEC), c0 = (c % (XC / VEC)) * VEC;
      const int j = jb + c0;  // 16-byte chunks are wholly in or out of [0, LkP)
      if (c < XV && j >= 0 && j < bp.f.LkP) {
        xr[k] = *reinterpret_cast<const vecT*>(dsb + (int64_t)(i0 + r) * bp.f.LkP + j);
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) xr[k][e] = (T)0.0f;
      }
    }
    const T* qbase = (const T*)p.q + (int64_t)b * p.qs[0] + (int64_t)h * p.qs[2];
    const T* kbase = (const T*)p.k + (int64_t)b * p.ks[0] + (int64_t)h * p.ks[2];
#pragma unroll
    for (int k = 0; k < RCH; ++k) {
      const int c = tid + 256 * k;
      const int r = c / (D / VEC), c0 = (c % (D / VEC)) * VEC;
      const int i = i0 + r, j = jb + XC - JC + r;  // the ring's new rows
#pragma unroll
      for (int e = 0; e < VEC; ++e) qr[k][e] = kr[k][e] = (T)0.0f;
      if (c < RV && c2p && i < p.Lq) qr[k] = *reinterpret_cast<const vecT*>(qbase + (int64_t)i * p.qs[1] + c0);
      if (c < RV && p2c && j >= 0 && j < p.Lk) kr[k] = *reinterpret_cast<const vecT*>(kbase + (int64_t)j * p.ks[1] + c0);
    }
  };

  if (nsteps > 0) fetch(0);
  for (int st = 0; st < nsteps; ++st) {
    int b, i0;
    step_coords(st, b, i0);
    const int jb = i0 - d0 - DBW;  // key of staged column 0
    __syncthreads();               // previous step's readers are done
#pragma unroll
    for (int k = 0; k < XCH; ++k) {
      const int c = tid + 256 * k;
      if (c < XV) {
        const int r = c / (XC / VEC), c0 = (c % (XC / VEC)) * VEC;
        *reinterpret_cast<vecT*>(Xs + (XP + r) * XSTR + c0) = xr[k];
      }
    }
#pragma unroll
    for (int k = 0; k < RCH; ++k) {
      const int c = tid + 256 * k;
      if (c < RV) {
        const int r = c / (D / VEC), c0 = (c % (D / VEC)) * VEC;
        *reinterpret_cast<vecT*>(Qc + r * KSTR + c0) = qr[k];
        *reinterpret_cast<vecT*>(Kring + ((jb + XC - JC + r) & (QRING - 1)) * RSTR + c0) = kr[k];
      }
    }
    if (p2c && i0 == istart) {  // first chunk of a batch: the ring's older rows too
      const T* kbase = (const T*)p.k + (int64_t)b * p.ks[0] + (int64_t)h * p.ks[2];
      load_ring_rows<T, D>(Kring, RSTR, kbase, p.ks[1], jb, XC - JC, p.Lk, tid);
    }
    __syncthreads();
    if (st + 1 < nsteps) fetch(st + 1);

    // A operands, shared by the wave's two 16-offset blocks: Q^T of the 32
    // queries, and K^T of staged columns [32w, 32w + 64).
    frag qa[GC_STEPS][ND], ka[GP_STEPS][ND];
    if (c2p) {
#pragma unroll
      for (int s = 0; s < GC_STEPS; ++s)
#pragma unroll
        for (int db = 0; db < ND; ++db) qa[s][db] = tr_contig<T>(Qc, KSTR, s * M::KSTEP, 16 * db, g, c16);
    }
    if (p2c) {
#pragma unroll
      for (int s = 0; s < GP_STEPS; ++s)
#pragma unroll
        for (int db = 0; db < ND; ++db)
          ka[s][db] = tr_contig_ring<T>(Kring, RSTR, jb, 32 * w + M::KSTEP * s, 16 * db, g, c16);
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int e0 = 16 * (2 * w + t);  // first e of this wave's 16-offset block
      if (c2p) {
        // Gc^T[d][e] += sum_r Q^T[d][i0 + r] X[r][r + 1 + e],  r = KSTEP*s + FE*g + u
#pragma unroll
        for (int s = 0; s < GC_STEPS; ++s) {
          frag bfr;
          const T* dg = Xs + (XP + M::KSTEP * s + FE * g) * XSTR + M::KSTEP * s + FE * g + 1 + e0 + c16;
#pragma unroll
          for (int u = 0; u < FE; ++u) bfr[u] = dg[u * (XSTR + 1)];
#pragma unroll
          for (int db = 0; db < ND; ++db) gc[t][db] = M::mma(qa[s][db], bfr, gc[t][db]);
        }
      }
      if (p2c) {
        // Gp^T[d][e] += sum_c K^T[d][jb + c] X[c - 1 - e][c],  c = 32w + KSTEP*s + FE*g + u;
        // X rows c - 1 - e in [-32, 63) (zero outside [0, JC)).
#pragma unroll
        for (int s = 0; s < GP_STEPS; ++s) {
          frag bfr;
          const int c = 32 * w + M::KSTEP * s + FE * g;  // column of element u = 0
          const T* dg = Xs + (XP + c - 1 - e0 - c16) * XSTR + c;
#pragma unroll
          for (int u = 0; u < FE; ++u) bfr[u] = dg[u * (XSTR + 1)];
#pragma unroll
          for (int db = 0; db < ND; ++db) gp[t][db] = M::mma(ka[s][db], bfr, gp[t][db]);
        }
      }
    }
  }

  // partial of this (block, head, batch group): [type][dd][d], fp32
  float* out = bp.gpart + ((int64_t)(h * bp.NDB + dblk) * bp.NBG + bg) * 2 * DBW * D;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int dd = DBW - 1 - (16 * (2 * w + t) + c16);  // offset d0 + dd
#pragma unroll
    for (int db = 0; db < ND; ++db) {
      *reinterpret_cast<f32x4*>(out + (int64_t)dd * D + 16 * db + 4 * g) = gc[t][db];
      *reinterpret_cast<f32x4*>(out + (int64_t)(DBW + dd) * D + 16 * db + 4 * g) = gp[t][db];
    }
  }
}

// tab[h][r][:] (+)= s * sum over batch groups and offsets d with row(d) = r
// of the partials (accumulated into fp32, or written in fp32 or bf16).  One
// wave per (table, h, r): 64 / (D/4) parts split the row's offset range
// [begin, end) (from dsa_bwd_segments_kernel) and are summed with lane
// shuffles; lanes of a part hold 4 columns each.
template <int D>
__global__ __launch_bounds__(64) void dsa_bwd_fold_kernel(BwdParams bp) {
  using namespace tbcfg;
  const FwdParams& p = bp.f;
  const int R = 2 * p.A;
  constexpr int Q4 = D / 4, NP = 64 / Q4;
  const int t = blockIdx.x / (p.H * R), h = (blockIdx.x / R) % p.H, r = blockIdx.x % R;
  if (!(p.flags & (1 << t))) return;
  const bool q = t == 1;  // false: dKr (c2p), true: dQr (p2c)
  const int c4 = threadIdx.x % Q4, part = threadIdx.x / Q4;
  const int beg = bp.seg[(2 * t) * R + r], end = bp.seg[(2 * t + 1) * R + r];
  f32x4 acc = zero4();
  for (int d = beg + part; d < end; d += NP) {
    const int dblk = (d + bp.f.LkP) / DBW, dd = (d + bp.f.LkP) % DBW;
    const float* src = bp.gpart + ((int64_t)(h * bp.NDB + dblk) * bp.NBG) * 2 * DBW * D +
                       (int64_t)((q ? DBW : 0) + dd) * D + 4 * c4;
    for (int k = 0; k < bp.NBG; ++k) acc += *reinterpret_cast<const f32x4*>(src + (int64_t)k * 2 * DBW * D);
  }
#pragma unroll
  for (int m = Q4; m < 64; m <<= 1)
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] += __shfl_xor(acc[e], m);
  if (part != 0) return;
  const int64_t o = ((int64_t)h * R + r) * D + 4 * c4;
  void* tab = q ? bp.dqr : bp.dkr;
  const f32x4 v = acc * p.scale;
  if (bp.dtab_bf16) {
    typedef bf16 b4 __attribute__((ext_vector_type(4)));
    *reinterpret_cast<b4*>((bf16*)tab + o) = b4{(bf16)v[0], (bf16)v[1], (bf16)v[2], (bf16)v[3]};
  } else if (bp.dtab_overwrite) {
    *reinterpret_cast<f32x4*>((float*)tab + o) = v;
  } else {
    f32x4* tp = reinterpret_cast<f32x4*>((float*)tab + o);
    *tp = *tp + v;
  }
}

}  // namespace dsa
