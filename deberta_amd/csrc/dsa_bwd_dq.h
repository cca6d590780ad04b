// dsa_bwd_dq.h — dQ and dKr of the fused disentangled attention (gfx950).
//
// Persistent grid: workgroup g walks the contiguous run of work items
// [g*N/G, (g+1)*N/G) where an item is (head h, batch b, 128-query tile) with
// the head slowest.  Per item it streams 64-key tiles and computes, per tile
// (4 waves x 32 queries):
//   scores        y = (K Q^T + c2p + p2c) * scale*log2e   (as the forward)
//   P, dP, dS     P = exp2(y - lse*log2e), dP = dO V^T, dS = P (dP - Delta)
//   dQ^T         += K^T dS^T                         (K^T read transposed from LDS)
//   dQ^T (c2p)   += KrW^T Ar,  dKr += Ar Q          (c2p, see below)
// c2p gradients: the wave's dS values are first stored by query/key offset,
// dSd[x][i] with x = (i - i0) - (j - j0) + 63 - 32w (a compile-time offset
// from a per-lane base).  The table row of offset x is c(x), non-decreasing
// in x, so the offsets of one table row r form a contiguous range X(r)
// (found by binary search in the tile's row table).  One pass folds dSd
// onto table rows without atomics, Ar[r][i] = sum_{x in X(r)} dSd[x][i], for
// the tile's window of at most 192 rows (wider windows are processed in
// chunks).  Then
//   dQ^T[d][i]  += sum_r KrW^T[d][r] Ar[r][i]   (both operands read
//                                               transposed from LDS)
//   dKr[r][d]   += sum_i Ar[r][i] Q[i][d]       (16-row blocks, owned by
//                                               wave (block % 4))
// with KrW the tile's window of Kr rows.  The register partial of a head is
// written once, when the workgroup moves to another head or finishes, to a
// per-workgroup slot of the workspace; dsa_bwd_reduce_kernel adds the slots
// into dKr.
#pragma once

#include "dsa_tiles.h"

namespace dsa {

namespace dqcfg {
constexpr int NW = 4, WQ = 32, BQ = 128, BK = 64;
constexpr int XW = 96;       // offset rows per wave
constexpr int XG = 192;      // offset rows per workgroup
constexpr int DS2 = 40;      // dSd row stride (elements): [x][i], 32 queries + pad
constexpr int AR_ROWS = 192; // table rows per folded band chunk (bf16; 64 for fp32)
constexpr int AR_STR = 136;  // folded band row stride (elements): [r][i], 128 queries + pad
constexpr int OWN = 8;       // register-held 16-row table blocks per wave (rows < 512)
}  // namespace dqcfg

// Number of items, slots per workgroup and partial rows of the persistent
// backward kernels (shared with the host).
struct PersistentPlan {
  int items;      // H * B * tiles
  int per_head;   // B * tiles
  int grid;       // workgroups
  int slots;      // partial slots per workgroup (heads a workgroup can span)
  int prow;       // partial rows (min(R, 512))
};

DSA_DEV int item_begin(int g, int items, int grid) { return (int)(((int64_t)g * items) / grid); }

// Adds one 16 x D block (C layout: col d = 16*db + c16, rows r0 + 4g + e) of
// a table gradient to fp32 global memory with atomics (rows >= R skipped).
template <int D>
DSA_DEV void atomic_rows(float* tab, int R, int r0, const f32x4 (&v)[D / 16], int g, int c16) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int r = r0 + 4 * g + e;
    if (r < R) {
#pragma unroll
      for (int db = 0; db < D / 16; ++db) atomicAdd(tab + (int64_t)r * D + 16 * db + c16, v[db][e]);
    }
  }
}

// Writes the register-owned partial of one head (rows < prow) to its slot.
template <int D>
DSA_DEV void store_partial(float* slot, int prow, const f32x4 (&acc)[dqcfg::OWN][D / 16], float scale, int w,
                           int g, int c16) {
#pragma unroll
  for (int k = 0; k < dqcfg::OWN; ++k) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int r = 16 * (dqcfg::NW * k + w) + 4 * g + e;
      if (r < prow) {
#pragma unroll
        for (int db = 0; db < D / 16; ++db) slot[(int64_t)r * D + 16 * db + c16] = acc[k][db][e] * scale;
      }
    }
  }
}

// KrW[r - r0] = Kr[r] for r in [r0, r1] (r < R), zero for the rest of the
// AR_ROWS-row window.
template <typename T, int D>
DSA_DEV void stage_kr_window(T* KrW, int str, const T* krh, int64_t krs, int r0, int r1, int R, int tid) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int CPR = D / VEC;
  constexpr int ROWS = sizeof(T) == 2 ? dqcfg::AR_ROWS : 64;
  typedef T vecT __attribute__((ext_vector_type(VEC)));
  for (int c = tid; c < ROWS * CPR; c += 256) {
    const int rr = c / CPR, d0 = (c % CPR) * VEC;
    const int r = r0 + rr;
    vecT v;
    if (r <= r1 && r < R) {
      v = *reinterpret_cast<const vecT*>(krh + (int64_t)r * krs + d0);
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) v[e] = (T)0.0f;
    }
    *reinterpret_cast<vecT*>(KrW + rr * str + d0) = v;
  }
}

template <typename T, int D, int MASK>
__global__ __launch_bounds__(256, 1) void dsa_bwd_dq_kernel(BwdParams bp, PersistentPlan plan, float* part) {
  using namespace dqcfg;
  using M = Mfma<T>;
  typedef typename M::frag frag;
  typedef typename BandType<T>::type BT;
  constexpr int NS = D / M::KSTEP;
  constexpr int ND = D / 16;
  constexpr bool BF = sizeof(T) == 2;
  constexpr int KSTR = D + Pad<T>::v;
  constexpr int BANDS_BYTES = (NW * dcfg::CB_ELEMS + dcfg::PB_ELEMS) * (int)sizeof(BT);
  constexpr int XW_ROWS = XW;
  constexpr int ARN = BF ? AR_ROWS : 64;  // table rows per folded chunk
  constexpr int DSD_BYTES = ((NW * XW_ROWS * DS2 * (int)sizeof(T) + 15) / 16) * 16;
  constexpr int AR_BYTES = ARN * AR_STR * (int)sizeof(T);
  constexpr int UNI_BYTES = (BANDS_BYTES > DSD_BYTES + AR_BYTES) ? BANDS_BYTES : DSD_BYTES + AR_BYTES;
  const FwdParams& p = bp.f;

  __shared__ __align__(16) T Ks[BK * KSTR];
  __shared__ __align__(16) T Vs[BK * KSTR];
  __shared__ __align__(16) T Qs[BF ? BQ * KSTR : 8];
  __shared__ __align__(16) T KrW[ARN * KSTR];
  __shared__ short crow[XG], prow[XG];
  __shared__ short xlo[AR_ROWS], xhi[AR_ROWS];
  __shared__ __align__(16) char uni[UNI_BYTES];

  const int tid = threadIdx.x;
  const int w = tid >> 6, g = (tid & 63) >> 4, c16 = tid & 15;
  const int Lq = p.Lq, Lk = p.Lk, A = p.A, R = 2 * A;
  const bool c2p = (p.flags & 1) != 0;
  BT* cbw = reinterpret_cast<BT*>(uni) + w * dcfg::CB_ELEMS;
  BT* pbs = reinterpret_cast<BT*>(uni) + NW * dcfg::CB_ELEMS;
  T* dsd_all = reinterpret_cast<T*>(uni);
  T* dsd = dsd_all + w * XW_ROWS * DS2;
  T* Ar = reinterpret_cast<T*>(uni + DSD_BYTES);
  const float sl2 = p.scale * kLog2e;
  const int QT = (Lq + BQ - 1) / BQ;
  const int nkt = (Lk + BK - 1) / BK;

  f32x4 dkra[OWN][ND];
#pragma unroll
  for (int k = 0; k < OWN; ++k)
#pragma unroll
    for (int db = 0; db < ND; ++db) dkra[k][db] = zero4();
  int cur_h = -1, slot = 0;
  const int it0 = item_begin(blockIdx.x, plan.items, plan.grid);
  const int it1 = item_begin(blockIdx.x + 1, plan.items, plan.grid);

  for (int item = it0; item < it1; ++item) {
    const int h = item / plan.per_head;
    const int b = (item % plan.per_head) / QT;
    const int qt = item % QT;
    if (h != cur_h) {
      if (cur_h >= 0 && c2p) {
        store_partial<D>(part + ((int64_t)blockIdx.x * plan.slots + slot) * plan.prow * D, plan.prow, dkra, p.scale,
                         w, g, c16);
        ++slot;
      }
#pragma unroll
      for (int k = 0; k < OWN; ++k)
#pragma unroll
        for (int db = 0; db < ND; ++db) dkra[k][db] = zero4();
      cur_h = h;
    }
    const int i0 = qt * BQ;
    const int iw = i0 + w * WQ;
    const T* qbase = (const T*)p.q + (int64_t)b * p.qs[0] + (int64_t)h * p.qs[2];
    const T* kbase = (const T*)p.k + (int64_t)b * p.ks[0] + (int64_t)h * p.ks[2];
    const T* vbase = (const T*)p.v + (int64_t)b * p.vs[0] + (int64_t)h * p.vs[2];
    const T* dobase = (const T*)bp.dout + (int64_t)b * bp.dos[0] + (int64_t)h * bp.dos[2];
    const T* krh = c2p ? (const T*)p.kr + (int64_t)h * p.krs[0] : nullptr;
    const T* qrh = (p.flags & 2) ? (const T*)p.qr + (int64_t)h * p.qrs[0] : nullptr;
    const uint8_t* kkb = (MASK == MASK_KEY) ? p.kk + (int64_t)b * p.kkb : nullptr;
    const uint8_t* pkb = (MASK == MASK_PAIR) ? p.pk + (int64_t)b * p.pkb : nullptr;
    const float* lseb = p.lse + ((int64_t)b * p.H + h) * Lq;
    const float* dltb = bp.delta + ((int64_t)b * p.H + h) * Lq;

    int irow[2];
    bool ilive[2];
    float lse2[2], dlt[2];
    frag qf[2][NS], dof[2][NS];
#pragma unroll
    for (int ib = 0; ib < 2; ++ib) {
      const int i = iw + 16 * ib + c16;
      irow[ib] = i;
      const bool valid = i < Lq;
      bool live = valid;
      if (MASK == MASK_KEY && valid) live = kkb[i] != 0;
      if (MASK == MASK_PAIR && valid) live = pkb[(int64_t)i * p.pkq + i] != 0;
      ilive[ib] = live;
      lse2[ib] = live ? lseb[i] * kLog2e : INFINITY;
      dlt[ib] = valid ? dltb[i] : 0.f;
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        qf[ib][s] = valid ? M::load_contig(qbase + (int64_t)i * p.qs[1], s, g) : M::zero();
        dof[ib][s] = valid ? M::load_contig(dobase + (int64_t)i * bp.dos[1], s, g) : M::zero();
      }
    }

    // Q rows of the item in LDS (B operand of the dKr product), then the
    // per-item fragments of this wave's 32 query rows.
    __syncthreads();  // previous item's LDS use is over
    if constexpr (BF) {
      if (c2p) load_rows<T, D, BQ, 256>(Qs, KSTR, nullptr, 0, qbase, p.qs[1], i0, Lq, tid);
    }
    int wg_live = 0;
    if (tid < BQ) {
      const int i = i0 + tid;
      if (i < Lq) {
        if (MASK == MASK_NONE) wg_live = 1;
        else if (MASK == MASK_KEY) wg_live = kkb[i] != 0;
        else wg_live = pkb[(int64_t)i * p.pkq + i] != 0;
      }
    }
    const bool any_live = __syncthreads_or(wg_live);
    f32x4 dqa[ND][2];
#pragma unroll
    for (int db = 0; db < ND; ++db) dqa[db][0] = dqa[db][1] = zero4();

    for (int kt = 0; any_live && kt < nkt; ++kt) {
      const int j0 = kt * BK;
      if (MASK == MASK_KEY) {
        int keep = 0;
        if (tid < BK) keep = (j0 + tid < Lk) && kkb[j0 + tid];
        if (!__syncthreads_or(keep)) continue;
      } else if (MASK == MASK_PAIR) {
        int keep = 0;
        const int r = tid >> 1, half = tid & 1;
        const int i = i0 + r;
        if (i < Lq) {
          const uint8_t* row = pkb + (int64_t)i * p.pkq;
          const int jb0 = j0 + half * (BK / 2);
          const int jend = min(jb0 + BK / 2, Lk);
          for (int j = jb0; j < jend; ++j) keep |= row[j];
        }
        if (!__syncthreads_or(keep)) continue;
      }
      __syncthreads();
      load_rows<T, D, BK, 256>(Ks, KSTR, nullptr, 0, kbase, p.ks[1], j0, Lk, tid);
      load_rows<T, D, BK, 256>(Vs, KSTR, nullptr, 0, vbase, p.vs[1], j0, Lk, tid);
      if (p.flags) load_row_tables(crow, prow, p.rel, i0, j0, Lq, Lk, A, tid);
      // Window of Kr rows [c(x=0), c(x=0) + 192) for the c2p band and the dQ
      // product; "fast" when the tile's table rows fit it (always for tables
      // with unit steps, the reference's log buckets included).
      int wide = 0;
      if (c2p) {
        const int r0 = c2p_row(min(max(p.rel[min(max(i0 - j0 - (BK - 1), -(Lk - 1)), Lq - 1) + Lk - 1], -A), A), A);
        const int r1 = c2p_row(min(max(p.rel[min(max(i0 - j0 + BQ, -(Lk - 1)), Lq - 1) + Lk - 1], -A), A), A);
        wide = (r1 - r0 + 1 > ARN) ? 1 : 0;
        if (!wide) stage_kr_window<T, D>(KrW, KSTR, krh, p.krs[1], r0, r1, R, tid);
      }
      const bool fast = !__syncthreads_or(wide);

      // ---- recompute scores (log2 domain, as the forward) ----------------------
      frag kf[4][NS];
#pragma unroll
      for (int jb = 0; jb < 4; ++jb)
#pragma unroll
        for (int s = 0; s < NS; ++s) kf[jb][s] = M::load_contig(&Ks[(16 * jb + c16) * KSTR], s, g);
      f32x4 st[2][4];
#pragma unroll
      for (int jb = 0; jb < 4; ++jb)
#pragma unroll
        for (int ib = 0; ib < 2; ++ib) {
          f32x4 acc = zero4();
#pragma unroll
          for (int s = 0; s < NS; ++s) acc = M::mma(kf[jb][s], qf[ib][s], acc);
          st[ib][jb] = acc * sl2;
        }
      if (p.flags)
        add_delta_bands_T<T, D>(st, kf, qf, cbw, pbs, crow, prow, w, g, c16, krh, p.krs[1], qrh, p.qrs[1], p.flags,
                                sl2, (c2p && fast) ? (const T*)KrW : nullptr, KSTR, (c2p && fast) ? crow[0] : 0);

      // ---- P^T, dP^T, dS^T -------------------------------------------------------
      f32x4 ds[2][4];
#pragma unroll
      for (int jb = 0; jb < 4; ++jb) {
        frag vf[NS];
#pragma unroll
        for (int s = 0; s < NS; ++s) vf[s] = M::load_contig(&Vs[(16 * jb + c16) * KSTR], s, g);
#pragma unroll
        for (int ib = 0; ib < 2; ++ib) {
          f32x4 dp = zero4();
#pragma unroll
          for (int s = 0; s < NS; ++s) dp = M::mma(vf[s], dof[ib][s], dp);
          const int i = irow[ib];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int j = j0 + 16 * jb + 4 * g + e;
            bool keep = ilive[ib] && j < Lk;
            if (MASK == MASK_KEY) keep = keep && kkb[j] != 0;
            if (MASK == MASK_PAIR) keep = keep && pkb[(int64_t)i * p.pkq + j] != 0;
            const float pe = keep ? exp2f(st[ib][jb][e] - lse2[ib]) : 0.f;
            ds[ib][jb][e] = pe * (dp[e] - dlt[ib]);
          }
        }
      }

      // ---- dQ^T += K^T dS^T (K^T read transposed from the K tile) --------------------
#pragma unroll
      for (int s = 0; s < BK / M::KSTEP; ++s) {
        frag df[2];
#pragma unroll
        for (int ib = 0; ib < 2; ++ib) df[ib] = M::from_acc(ds[ib], s);
#pragma unroll
        for (int db = 0; db < ND; ++db) {
          const frag ktf = tr_acc<T>(Ks, KSTR, s * M::KSTEP, 16 * db, g, c16);
#pragma unroll
          for (int ib = 0; ib < 2; ++ib) dqa[db][ib] = M::mma(ktf, df[ib], dqa[db][ib]);
        }
      }

      if (c2p) {
        const int rlo = crow[0];
        const int nr = crow[XG - 1] - rlo + 1;  // rows of the tile's window (row table is monotone)
        __syncthreads();  // score bands are consumed; the union region is free
        // dS^T -> dSd[x][i] (this wave's block), x = i_local - j_local + 63
        {
          constexpr int DSD_V = XW_ROWS * DS2 * (int)sizeof(T) / 16;
          f32x4* z = reinterpret_cast<f32x4*>(dsd);
          for (int x = (tid & 63); x < DSD_V; x += 64) z[x] = zero4();
          wave_lds_sync();
          T* base = dsd + (c16 - 4 * g + 63) * DS2 + c16;
#pragma unroll
          for (int ib = 0; ib < 2; ++ib)
#pragma unroll
            for (int jb = 0; jb < 4; ++jb)
#pragma unroll
              for (int e = 0; e < 4; ++e) base[(16 * ib - 16 * jb - e) * DS2 + 16 * ib] = (T)ds[ib][jb][e];
        }
        for (int cb = rlo; cb < rlo + nr; cb += ARN) {
          const int ncr = min(ARN, rlo + nr - cb);
          if (!fast) {
            __syncthreads();  // previous chunk's readers of KrW / Ar are done
            stage_kr_window<T, D>(KrW, KSTR, krh, p.krs[1], cb, cb + ncr - 1, R, tid);
          }
          // offsets of each table row of the chunk: X(r) = [xlo, xhi]
          if (tid < ARN) {
            const int r = cb + tid;
            int lo = 0, hi = XG;
            while (lo < hi) {  // first x with crow[x] >= r
              const int mid = (lo + hi) >> 1;
              if (crow[mid] < r) lo = mid + 1; else hi = mid;
            }
            int lo2 = lo, hi2 = XG;
            while (lo2 < hi2) {  // first x with crow[x] > r
              const int mid = (lo2 + hi2) >> 1;
              if (crow[mid] <= r) lo2 = mid + 1; else hi2 = mid;
            }
            xlo[tid] = (short)lo;
            xhi[tid] = (short)(lo2 - 1);
          }
          __syncthreads();
          // fold: Ar[r][i] = sum_{x in X(r)} dSd[x][i]
          for (int q = tid; q < ARN * (BQ / 8); q += 256) {
            const int rr = q >> 4, c = q & 15;
            const int ws = c >> 2, il = 8 * c - WQ * ws;
            float acc[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[e] = 0.f;
            if (rr < ncr) {
              const int x1 = xhi[rr];
              for (int x = xlo[rr]; x <= x1; ++x) {
                const int xl = x - WQ * ws;
                if (xl >= 0 && xl < XW_ROWS) {
                  const T* src = dsd_all + (ws * XW_ROWS + xl) * DS2 + il;
                  if constexpr (BF) {
                    const bf16x8 v = *reinterpret_cast<const bf16x8*>(src);
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc[e] += (float)v[e];
                  } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc[e] += src[e];
                  }
                }
              }
            }
            T* dst = Ar + rr * AR_STR + 8 * c;
            if constexpr (BF) {
              bf16x8 o;
#pragma unroll
              for (int e = 0; e < 8; ++e) o[e] = (bf16)acc[e];
              *reinterpret_cast<bf16x8*>(dst) = o;
            } else {
#pragma unroll
              for (int e = 0; e < 8; ++e) dst[e] = acc[e];
            }
          }
          __syncthreads();
          // dQ^T[d][i] += sum_r KrW^T[d][r] Ar[r][i]   (this wave's 32 queries)
          const int nsteps = (ncr + M::KSTEP - 1) / M::KSTEP;
          for (int s = 0; s < nsteps; ++s) {
            frag bfr[2];
#pragma unroll
            for (int ib = 0; ib < 2; ++ib) bfr[ib] = tr_contig<T>(Ar, AR_STR, s * M::KSTEP, WQ * w + 16 * ib, g, c16);
#pragma unroll
            for (int db = 0; db < ND; ++db) {
              const frag af = tr_contig<T>(KrW, KSTR, s * M::KSTEP, 16 * db, g, c16);
#pragma unroll
              for (int ib = 0; ib < 2; ++ib) dqa[db][ib] = M::mma(af, bfr[ib], dqa[db][ib]);
            }
          }
          // dKr[r][d] += sum_i Ar[r][i] Q[i][d]   (16-row blocks this wave owns)
          const int blo = cb >> 4, bhi = (cb + ncr - 1) >> 4;
          for (int rb = blo + ((w - blo % NW) + NW) % NW; rb <= bhi; rb += NW) {
            const int rr = 16 * rb + c16 - cb;
            const bool rok = rr >= 0 && rr < ncr;
            f32x4 res[ND];
#pragma unroll
            for (int db = 0; db < ND; ++db) res[db] = zero4();
#pragma unroll
            for (int s = 0; s < BQ / M::KSTEP; ++s) {
              const frag af = rok ? M::load_contig(Ar + rr * AR_STR, s, g) : M::zero();
#pragma unroll
              for (int db = 0; db < ND; ++db) {
                frag bq;
                if constexpr (BF) {
                  bq = tr_contig<T>(Qs, KSTR, s * M::KSTEP, 16 * db, g, c16);
                } else {
#pragma unroll
                  for (int e = 0; e < 4; ++e) {
                    const int i = i0 + s * M::KSTEP + 4 * g + e;
                    bq[e] = (i < Lq) ? qbase[(int64_t)i * p.qs[1] + 16 * db + c16] : 0.f;
                  }
                }
                res[db] = M::mma(af, bq, res[db]);
              }
            }
            const int k = rb / NW;
            bool held = false;
#pragma unroll
            for (int kk = 0; kk < OWN; ++kk) {
              if (k == kk) {
#pragma unroll
                for (int db = 0; db < ND; ++db) dkra[kk][db] += res[db];
                held = true;
              }
            }
            if (!held) {
#pragma unroll
              for (int db = 0; db < ND; ++db) res[db] *= p.scale;
              atomic_rows<D>(bp.dkr + (int64_t)h * R * D, R, 16 * rb, res, g, c16);
            }
          }
        }
      }
    }

    // ---- dQ of the item ---------------------------------------------------------------
    T* dqbase = (T*)bp.dq + (int64_t)b * bp.dqs[0] + (int64_t)h * bp.dqs[2];
#pragma unroll
    for (int ib = 0; ib < 2; ++ib) {
      const int i = irow[ib];
      if (i < Lq) {
        T* row = dqbase + (int64_t)i * bp.dqs[1];
#pragma unroll
        for (int db = 0; db < ND; ++db) {
          typedef T vec4 __attribute__((ext_vector_type(4)));
          vec4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = (T)(dqa[db][ib][e] * p.scale);
          *reinterpret_cast<vec4*>(row + 16 * db + 4 * g) = v;
        }
      }
    }
  }
  if (cur_h >= 0 && c2p) {
    store_partial<D>(part + ((int64_t)blockIdx.x * plan.slots + slot) * plan.prow * D, plan.prow, dkra, p.scale, w, g,
                     c16);
  }
}

// tab[h, r, d] += sum of the partial slots written for head h (r < prow).
template <int D>
__global__ __launch_bounds__(256) void dsa_bwd_reduce_kernel(float* tab, const float* part, PersistentPlan plan,
                                                             int H, int R) {
  const int64_t n = (int64_t)H * plan.prow * D;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= n) return;
  const int h = (int)(idx / ((int64_t)plan.prow * D));
  const int64_t rd = idx % ((int64_t)plan.prow * D);
  const int first = h * plan.per_head, last = (h + 1) * plan.per_head;  // item range of the head
  // workgroups whose item runs intersect [first, last)
  int g0 = (int)(((int64_t)first * plan.grid) / plan.items) - 1;
  if (g0 < 0) g0 = 0;
  float acc = 0.f;
  for (int g = g0; g < plan.grid; ++g) {
    const int a = item_begin(g, plan.items, plan.grid), b = item_begin(g + 1, plan.items, plan.grid);
    if (a >= last) break;
    if (b <= first || a == b) continue;
    const int slot = h - a / plan.per_head;
    acc += part[((int64_t)g * plan.slots + slot) * plan.prow * D + rd];
  }
  tab[(int64_t)h * R * D + rd] += acc;
}

}  // namespace dsa
