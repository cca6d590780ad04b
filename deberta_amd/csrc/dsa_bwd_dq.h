// dsa_bwd_dq.h — dQ of the fused disentangled attention from the stored dS
// (gfx950).
//
// One workgroup = 4 waves = one (batch b, head h, 128-query tile); wave w
// owns queries [i0 + 32w, i0 + 32w + 32) and streams 64-key tiles of dS
// (rows = queries), K and the tile's krgt window through LDS (fetched into
// registers two tiles ahead):
//   dQ^T[d][i] += sum_j K^T[d][j] dS[i][j]              (K^T read transposed,
//                                                        dS rows contiguous)
//   dQ^T[d][i] += sum_x krgt[d][t0 + x] E[x][i]          (c2p)
// where x = (i - iw) - (j - j0) + 63 is the wave's offset index, E[x][i] =
// dS(i, j), and krgt holds the Kr rows gathered per offset and transposed.
// For one query, consecutive x are consecutive keys (descending), so E's
// operand is eight consecutive elements of one staged dS row; krgt stores
// each aligned group of eight offsets reversed, so the A operand's k order
// matches (ascending keys).  32 zero columns before each staged row (and
// the next row's, after it) cover offsets outside the tile.  No softmax
// state is needed: dS holds zeros for masked pairs and dead rows.
#pragma once

#include "dsa_bwd.h"

namespace dsa {

namespace dqcfg {
constexpr int NW = 4, WQ = 32, BQ = 128, BK = 64;
constexpr int MAX_KT = 1024;  // key tiles (Lk <= 65536)
constexpr int XW = 96;   // offset rows per wave (95 used)
constexpr int ZC = 32;   // zero columns before each staged dS row
}  // namespace dqcfg

// LDS of a dq workgroup (a struct, so that the kernel that runs dq and table
// workgroups in one launch can overlay it with the table kernel's).
template <typename T, int D>
struct DqLds {
  static constexpr int SSTR = sizeof(T) == 2 ? 104 : 100;  // staged dS row stride (see dq_body)
  static constexpr int GSTR = dqcfg::BQ + dqcfg::XW - dqcfg::WQ + Pad<T>::v;
  static constexpr int KSTR = D + Pad<T>::v;
  alignas(16) T Ss[(dqcfg::BQ + 1) * SSTR];
  alignas(16) T Ks[dqcfg::BK * KSTR];
  alignas(16) T KG[D * GSTR];
  short klist[dqcfg::MAX_KT];  // key tiles that can hold nonzero dS
  int segred[1];
};

// Workgroup blk of nblk (the logical index, whose remainder mod 8 is the
// XCD it runs on).  QC: the c2p part (the gradient of the c2p term's query
// rows qc) is accumulated apart and written to dqc; dq then holds the
// content part.
template <typename T, int D, bool QC>
DSA_DEV void dq_body(const BwdParams& bp, int blk, int nblk, DqLds<T, D>& L) {
  using namespace dqcfg;
  using M = Mfma<T>;
  typedef typename M::frag frag;
  constexpr int VEC = 16 / sizeof(T);
  typedef T vecT __attribute__((ext_vector_type(VEC)));
  constexpr int ND = D / 16;
  constexpr int FE = M::FRAG_ELEMS;               // k indices per lane per step
  static_assert(FE == VEC, "a fragment is one 16-byte chunk");
  constexpr int KSTR = DqLds<T, D>::KSTR;          // K tile row stride
  // Staged dS row: ZC zeros, BK keys, zeros up to the stride, and then the
  // next row's leading zeros; the stride makes 16 rows' 16-byte reads hit
  // distinct banks.  The c2p walk reads key columns [BK - XW, WQ + BK - 2].
  constexpr int SSTR = DqLds<T, D>::SSTR;
  static_assert(ZC + BK - XW >= 0 && WQ + BK - 2 < SSTR && ZC + BK <= SSTR, "zero columns cover the walk");
  constexpr int GW = BQ + XW - WQ;                // krgt columns of the workgroup's window (192)
  constexpr int GSTR = DqLds<T, D>::GSTR;
  static_assert(GSTR == GW + Pad<T>::v, "krgt window stride");
  constexpr int SV = BQ * BK / VEC, KV = BK * D / VEC, GV = D * GW / VEC;  // 16-byte chunks per tile
  constexpr int SCH = (SV + 255) / 256, KCH = (KV + 255) / 256, GCH = (GV + 255) / 256;
  const FwdParams& p = bp.f;

  T* const Ss = L.Ss;
  T* const Ks = L.Ks;
  T* const KG = L.KG;
  short* const klist = L.klist;
  int* const segred = L.segred;

  const int tid = threadIdx.x;
  const int w = tid >> 6, g = (tid & 63) >> 4, c16 = tid & 15;
  const int NQT = bp.f.LqP / BQ;
  // (b, h, qt), qt fastest; with an order (masks), item order[r / H] and
  // head r % H, heaviest first
  int qt, h, b;
  if (bp.qorder) {
    const int it = bp.qorder[blk / p.H];
    h = blk % p.H, qt = it % NQT, b = it / NQT;
  } else {
    const int m = xcd_remap(blk, nblk);
    qt = m % NQT, h = (m / NQT) % p.H, b = m / (NQT * p.H);
  }
  const int i0 = qt * BQ, iw = i0 + w * WQ;
  const bool c2p = (p.flags & 1) != 0;
  const T* kbase = (const T*)p.k + (int64_t)b * p.ks[0] + (int64_t)h * p.ks[2];
  const T* dsb = (const T*)bp.ds + ((int64_t)(b * p.H + h) * bp.f.LqP + i0) * bp.f.LkP;
  const T* krg = c2p ? (const T*)bp.krgt + (int64_t)h * D * bp.TGP : nullptr;

  // zeros everywhere; the key columns are overwritten per tile
  {
    vecT z;
#pragma unroll
    for (int e = 0; e < VEC; ++e) z[e] = (T)0.0f;
    static_assert((BQ + 1) * SSTR % VEC == 0, "whole chunks");
    for (int c = tid; c < (BQ + 1) * SSTR / VEC; c += 256) reinterpret_cast<vecT*>(Ss)[c] = z;
  }

  f32x4 dqa[ND][2];
#pragma unroll
  for (int db = 0; db < ND; ++db) dqa[db][0] = dqa[db][1] = zero4();
  f32x4 dqca[QC ? ND : 1][2];  // QC: the c2p part
#pragma unroll
  for (int db = 0; db < (QC ? ND : 1); ++db) dqca[db][0] = dqca[db][1] = zero4();

  // Key tiles (dS columns, K rows, krgt window) are fetched into registers
  // two tiles ahead, into two register sets used in turn (a tile's compute
  // alone is too short to cover the loads' latency).
  struct Regs {
    vecT s[SCH], k[KCH], g[GCH];
  };
  Regs ra, rb;
  auto fetch = [&](int entry, Regs& r) {
    vecT(&sr)[SCH] = r.s;
    vecT(&kr)[KCH] = r.k;
    vecT(&gr)[GCH] = r.g;
    const int kt = entry & 1023, cmask = entry >> 10;
    const int j0 = kt * BK;
#pragma unroll
    for (int k = 0; k < SCH; ++k) {
      const int c = tid + 256 * k;
      const int row = c / (BK / VEC);
#pragma unroll
      for (int e = 0; e < VEC; ++e) sr[k][e] = (T)0.0f;
      if (c < SV && ((cmask >> (row / 32)) & 1))
        // non-temporal: this kernel reads each dS element once, and the
        // table kernel's band reads (in the same launch) keep the lines
        // they share in the caches (full step 438 -> 427 us at the headline
        // shape with the saved term's copies in dkdv also non-temporal)
        sr[k] = __builtin_nontemporal_load(
            reinterpret_cast<const vecT*>(dsb + (int64_t)row * bp.f.LkP + j0 + (c % (BK / VEC)) * VEC));
    }
#pragma unroll
    for (int k = 0; k < KCH; ++k) {
      const int c = tid + 256 * k;
      const int j = j0 + c / (D / VEC);
#pragma unroll
      for (int e = 0; e < VEC; ++e) kr[k][e] = (T)0.0f;
      if (c < KV && j < p.Lk) kr[k] = *reinterpret_cast<const vecT*>(kbase + (int64_t)j * p.ks[1] + (c % (D / VEC)) * VEC);
    }
    if (c2p) {
      const int tw = i0 - j0 - 63 + bp.OFF;  // window column 0 (a multiple of 32)
#pragma unroll
      for (int k = 0; k < GCH; ++k) {
        const int c = tid + 256 * k;
        if (c < GV) gr[k] = *reinterpret_cast<const vecT*>(krg + (int64_t)(c / (GW / VEC)) * bp.TGP + tw + (c % (GW / VEC)) * VEC);
      }
    }
  };

  // With a key-padding or segment mask, dS was computed only for the tiles
  // of 32 queries x 128 keys whose segments can meet (ChunkRange): a key
  // tile is visited if one of its 4 query chunks is active, and the rows of
  // inactive chunks are read as zeros.  klist holds kt | (chunk mask << 10).
  int nkt = bp.f.LkP / BK;
  if (bp.cinfo) {
    // listed by wave 0, one key tile per lane
    if (tid < 64) {
      const int nch = bp.f.LqP / 32;
      const int4* ci = bp.cinfo + (int64_t)b * nch;
      int n = 0;
      for (int k0 = 0; k0 < nkt; k0 += 64) {
        const int kt = k0 + tid;
        int mask = 0;
        if (kt < nkt) {
          const ChunkRange kr = key_tile_range(ci, kt / 2, nch);
#pragma unroll
          for (int u = 0; u < BQ / 32; ++u) mask |= chunk_range(ci, i0 / 32 + u).meets(kr) ? (1 << u) : 0;
        }
        n = wave_append(mask != 0, (short)(kt | (mask << 10)), klist, n);
      }
      if (tid == 0) segred[0] = n;
    }
    __syncthreads();
    nkt = __builtin_amdgcn_readfirstlane(segred[0]);
  } else {
    for (int t = tid; t < nkt; t += 256) klist[t] = (short)(t | (0xf << 10));
    __syncthreads();
  }
  auto tile = [&](int n, Regs& r) {
    __syncthreads();  // previous tile's readers are done
#pragma unroll
    for (int k = 0; k < SCH; ++k) {
      const int c = tid + 256 * k;
      if (c < SV) *reinterpret_cast<vecT*>(Ss + (c / (BK / VEC)) * SSTR + ZC + (c % (BK / VEC)) * VEC) = r.s[k];
    }
#pragma unroll
    for (int k = 0; k < KCH; ++k) {
      const int c = tid + 256 * k;
      if (c < KV) *reinterpret_cast<vecT*>(Ks + (c / (D / VEC)) * KSTR + (c % (D / VEC)) * VEC) = r.k[k];
    }
    if (c2p) {
#pragma unroll
      for (int k = 0; k < GCH; ++k) {
        const int c = tid + 256 * k;
        if (c < GV) *reinterpret_cast<vecT*>(KG + (c / (GW / VEC)) * GSTR + (c % (GW / VEC)) * VEC) = r.g[k];
      }
    }
    __syncthreads();
    if (n + 2 < nkt) fetch(klist[n + 2], r);

    // ---- dQ^T += K^T dS^T: B = dS row i, keys KSTEP*s + FE*g + [0, FE) -----------------------
#pragma unroll
    for (int s = 0; s < BK / M::KSTEP; ++s) {
      frag bfr[2];
#pragma unroll
      for (int ib = 0; ib < 2; ++ib)
        bfr[ib] = *reinterpret_cast<const frag*>(Ss + (WQ * w + 16 * ib + c16) * SSTR + ZC + M::KSTEP * s + FE * g);
#pragma unroll
      for (int db = 0; db < ND; ++db) {
        const frag af = tr_contig<T>(Ks, KSTR, s * M::KSTEP, 16 * db, g, c16);
#pragma unroll
        for (int ib = 0; ib < 2; ++ib) dqa[db][ib] = M::mma(af, bfr[ib], dqa[db][ib]);
      }
    }

    // ---- c2p: dQ^T += krgt[t0 + x]^T E[x] ---------------------------------------------------
    if (c2p) {
      // krgt column of x = 0 for this wave: iw - j0 - 63 + OFF, i.e. window
      // column 32w.  Element e of the fragment whose first offset is
      // xb = KSTEP*s + FE*g holds offset x = xb + FE - 1 - e, i.e. key
      // column (i - iw) + BK - FE - xb + e.
#pragma unroll
      for (int s = 0; s < XW / M::KSTEP; ++s) {
        const int xb = M::KSTEP * s + FE * g;
        frag bfr[2];
#pragma unroll
        for (int ib = 0; ib < 2; ++ib) {
          const int il = 16 * ib + c16;  // i - iw
          const T* row = Ss + (WQ * w + il) * SSTR + ZC + il + BK - FE - xb;
          lds_read_elems<T, FE>(bfr[ib], row);
        }
#pragma unroll
        for (int db = 0; db < ND; ++db) {
          const frag af = *reinterpret_cast<const frag*>(KG + (16 * db + c16) * GSTR + WQ * w + xb);
#pragma unroll
          for (int ib = 0; ib < 2; ++ib) {
            if constexpr (QC) dqca[db][ib] = M::mma(af, bfr[ib], dqca[db][ib]);
            else dqa[db][ib] = M::mma(af, bfr[ib], dqa[db][ib]);
          }
        }
      }
    }
  };
  if (nkt > 0) fetch(klist[0], ra);
  if (nkt > 1) fetch(klist[1], rb);
  for (int n = 0; n < nkt; n += 2) {
    tile(n, ra);
    if (n + 1 < nkt) tile(n + 1, rb);
  }

  // ---- dQ ---------------------------------------------------------------------------------
  T* dqbase = (T*)bp.dq + (int64_t)b * bp.dqs[0] + (int64_t)h * bp.dqs[2];
#pragma unroll
  for (int ib = 0; ib < 2; ++ib) {
    const int i = iw + 16 * ib + c16;
    if (i < p.Lq) {
      T* row = dqbase + (int64_t)i * bp.dqs[1];
#pragma unroll
      for (int db = 0; db < ND; ++db) {
        typedef T vec4 __attribute__((ext_vector_type(4)));
        vec4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (T)(dqa[db][ib][e] * p.scale);
        *reinterpret_cast<vec4*>(row + 16 * db + 4 * g) = v;
      }
      if constexpr (QC) {
        T* crow = (T*)bp.dqc + (int64_t)b * bp.dqcs[0] + (int64_t)h * bp.dqcs[2] + (int64_t)i * bp.dqcs[1];
#pragma unroll
        for (int db = 0; db < ND; ++db) {
          typedef T vec4 __attribute__((ext_vector_type(4)));
          vec4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = (T)(dqca[db][ib][e] * p.scale);
          *reinterpret_cast<vec4*>(crow + 16 * db + 4 * g) = v;
        }
      }
    }
  }
}

template <typename T, int D, bool QC = false>
__global__ __launch_bounds__(256, 2) void dsa_bwd_dq_kernel(BwdParams bp) {
  __shared__ DqLds<T, D> L;
  dq_body<T, D, QC>(bp, blockIdx.x, gridDim.x, L);
}

}  // namespace dsa
