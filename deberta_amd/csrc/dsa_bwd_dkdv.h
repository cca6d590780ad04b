// dsa_bwd_dkdv.h — dK, dV and dQr of the fused disentangled attention (gfx950).
//
// Mirror of dsa_bwd_dq.h with the roles of queries and keys exchanged.
// Persistent grid over items (head h, batch b, 128-key tile), head slowest.
// Per item the workgroup (4 waves x 32 keys) streams 64-query tiles:
//   scores        y = (Q K^T + c2p + p2c) * scale*log2e, queries down / keys
//                 across: the c2p band (queries are shared by the waves) is
//                 computed once per workgroup, the p2c band per wave
//   P, dP, dS     P = exp2(y - lse*log2e), dP = dO V^T, dS = P (dP - Delta)
//   dV^T         += dO^T P,  dK^T += Q^T dS              (operands read
//                                                        transposed from LDS)
//   p2c gradients, via offsets: dS stored at dSd[x][j] with
//                 x = (i - i0) - (j - j0) + 127 - (96 - 32w); the p2c table row
//                 p(x) is non-increasing in x, so each row's offsets are a
//                 contiguous range and one pass folds dSd onto table rows,
//                 Ap[p][j] = sum_{x in X(p)} dSd[x][j], without atomics; then
//                 dK^T[d][j] += sum_p QrW^T[d][p] Ap[p][j]
//                 dQr[p][d]  += sum_j Ap[p][j] K[j][d]   (16-row blocks owned
//                                                         by wave block % 4)
// dQr partials are kept in registers per head and written to per-workgroup
// slots; dsa_bwd_reduce_kernel adds them into dQr.
#pragma once

#include "dsa_bwd_dq.h"

namespace dsa {

namespace kvcfg {
constexpr int NW = 4, WK = 32, BKW = 128, BQ = 64;
constexpr int XW = 96;            // offset rows per wave
constexpr int XG = 192;           // offset rows per workgroup
constexpr int CBS = XG + 5;       // shared c2p band row stride [i][x]
constexpr int PBS = WK + 1;       // per-wave p2c band row stride [x][j]
constexpr int CB_ELEMS = BQ * CBS;
constexpr int PB_ELEMS = XW * PBS;
constexpr int DS2 = 40;           // dSd row stride [x][j]
constexpr int AR_ROWS = 192, AR_STR = 136;
constexpr int OWN = 8;
}  // namespace kvcfg

// Row tables of offsets dbase + x, x in [0, 192).
DSA_DEV void load_row_tables_at(short* crow, short* prow, const int32_t* rel, int dbase, int Lq, int Lk, int A,
                                int tid) {
  if (tid < kvcfg::XG) {
    int d = min(max(dbase + tid, -(Lk - 1)), Lq - 1);
    const int t = min(max(rel[d + Lk - 1], -A), A);
    crow[tid] = (short)c2p_row(t, A);
    prow[tid] = (short)p2c_row(t, A);
  }
}

// Adds the scaled c2p + p2c terms to a score tile in natural orientation
// (queries down, keys across; y[jb][ib][e] = query 16*ib + 4*g + e, key
// 32*w + 16*jb + c16 of the tile).  y holds (q.k) * scale*log2e.
//   qa: A fragments of the 64 query rows, kb: B fragments of the wave's keys
//   cbs: shared c2p band (BQ * CBS), pbw: this wave's p2c band (XW * PBS)
//   qrw: optional LDS window of Qr rows (row p at p - qrw_row0)
// Contains one __syncthreads.
template <typename T, int D>
DSA_DEV void add_delta_bands_S(f32x4 (&y)[2][4], const typename Mfma<T>::frag (&qa)[4][D / Mfma<T>::KSTEP],
                               const typename Mfma<T>::frag (&kb)[2][D / Mfma<T>::KSTEP],
                               typename BandType<T>::type* cbs, typename BandType<T>::type* pbw, const short* crow,
                               const short* prow, int w, int g, int c16, const T* krh, int64_t krs, const T* qrh,
                               int64_t qrs, int flags, float sl2, const T* qrw, int qrw_str, int qrw_row0) {
  using M = Mfma<T>;
  typedef typename M::frag frag;
  typedef typename BandType<T>::type BT;
  using namespace kvcfg;
  constexpr int NS = D / M::KSTEP;
  if (flags & 1) {  // shared c2p band: CB[i][x] = q_i . Kr[c(x)], wave w takes x-blocks w, w+4, w+8
#pragma unroll
    for (int t = 0; t < XG / 16 / NW; ++t) {
      const int xb = w + NW * t;
      const int row = crow[16 * xb + c16];
      frag bf[NS];
#pragma unroll
      for (int s = 0; s < NS; ++s) bf[s] = M::load_contig(krh + (int64_t)row * krs, s, g);
#pragma unroll
      for (int ib = 0; ib < 4; ++ib) {
        f32x4 acc = zero4();
#pragma unroll
        for (int s = 0; s < NS; ++s) acc = M::mma(qa[ib][s], bf[s], acc);
#pragma unroll
        for (int e = 0; e < 4; ++e) cbs[(16 * ib + 4 * g + e) * CBS + 16 * xb + c16] = to_band<BT>(acc[e] * sl2);
      }
    }
  }
  if (flags & 2) {  // per-wave p2c band: PB[x][j] = Qr[p(x)] . k_j, x over the wave's window
    const int xw0 = XW - WK * w;
#pragma unroll
    for (int xb = 0; xb < XW / 16; ++xb) {
      frag af[NS];
      if (qrw) {
        const int row = prow[xw0 + 16 * xb + c16] - qrw_row0;
#pragma unroll
        for (int s = 0; s < NS; ++s) af[s] = M::load_contig(qrw + row * qrw_str, s, g);
      } else {
        const int row = prow[min(xw0 + 16 * xb + c16, XG - 1)];
#pragma unroll
        for (int s = 0; s < NS; ++s) af[s] = M::load_contig(qrh + (int64_t)row * qrs, s, g);
      }
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) {
        f32x4 acc = zero4();
#pragma unroll
        for (int s = 0; s < NS; ++s) acc = M::mma(af[s], kb[jb][s], acc);
#pragma unroll
        for (int e = 0; e < 4; ++e) pbw[(16 * xb + 4 * g + e) * PBS + 16 * jb + c16] = to_band<BT>(acc[e] * sl2);
      }
    }
  }
  __syncthreads();
  if (flags & 1) {
    // i_local = 16*ib + 4*g + e, x = i_local - (32w + 16*jb + c16) + 127
    const BT* base = cbs + 4 * g * CBS + 4 * g - WK * w - c16 + 127;
#pragma unroll
    for (int jb = 0; jb < 2; ++jb)
#pragma unroll
      for (int ib = 0; ib < 4; ++ib)
#pragma unroll
        for (int e = 0; e < 4; ++e) y[jb][ib][e] += (float)base[(16 * ib + e) * CBS + 16 * ib + e - 16 * jb];
  }
  if (flags & 2) {
    // x_local = (16*ib + 4*g + e) - (16*jb + c16) + 31, column j_local = 16*jb + c16
    const BT* base = pbw + (4 * g - c16 + 31) * PBS + c16;
#pragma unroll
    for (int jb = 0; jb < 2; ++jb)
#pragma unroll
      for (int ib = 0; ib < 4; ++ib)
#pragma unroll
        for (int e = 0; e < 4; ++e) y[jb][ib][e] += (float)base[(16 * ib + e - 16 * jb) * PBS + 16 * jb];
  }
}

// QW[p - r0] = Qr[p] for p in [r0, r1] (p < R), zero for the rest of the window.
template <typename T, int D, int ROWS>
DSA_DEV void stage_rows_window(T* W, int str, const T* src, int64_t rs, int r0, int r1, int R, int tid) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int CPR = D / VEC;
  typedef T vecT __attribute__((ext_vector_type(VEC)));
  for (int c = tid; c < ROWS * CPR; c += 256) {
    const int rr = c / CPR, d0 = (c % CPR) * VEC;
    const int r = r0 + rr;
    vecT v;
    if (r <= r1 && r < R) {
      v = *reinterpret_cast<const vecT*>(src + (int64_t)r * rs + d0);
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) v[e] = (T)0.0f;
    }
    *reinterpret_cast<vecT*>(W + rr * str + d0) = v;
  }
}

template <typename T, int D, int MASK>
__global__ __launch_bounds__(256, 1) void dsa_bwd_dkdv_kernel(BwdParams bp, PersistentPlan plan, float* part) {
  using namespace kvcfg;
  using M = Mfma<T>;
  typedef typename M::frag frag;
  typedef typename BandType<T>::type BT;
  constexpr int NS = D / M::KSTEP;
  constexpr int ND = D / 16;
  constexpr bool BF = sizeof(T) == 2;
  constexpr int KSTR = D + Pad<T>::v;
  constexpr int ARN = BF ? AR_ROWS : 64;
  constexpr int BANDS_BYTES = (CB_ELEMS + NW * PB_ELEMS) * (int)sizeof(BT);
  constexpr int DSD_BYTES = ((NW * XW * DS2 * (int)sizeof(T) + 15) / 16) * 16;
  constexpr int AR_BYTES = ARN * AR_STR * (int)sizeof(T);
  constexpr int UNI_BYTES = (BANDS_BYTES > DSD_BYTES + AR_BYTES) ? BANDS_BYTES : DSD_BYTES + AR_BYTES;
  const FwdParams& p = bp.f;

  __shared__ __align__(16) T Qs[BQ * KSTR];
  __shared__ __align__(16) T dOs[BQ * KSTR];
  __shared__ __align__(16) T Ks[BF ? BKW * KSTR : 8];
  __shared__ __align__(16) T QrW[ARN * KSTR];
  __shared__ float rowv[2 * BQ];
  __shared__ short crow[XG], prow[XG];
  __shared__ short xlo[AR_ROWS], xhi[AR_ROWS];
  __shared__ __align__(16) char uni[UNI_BYTES];

  const int tid = threadIdx.x;
  const int w = tid >> 6, g = (tid & 63) >> 4, c16 = tid & 15;
  const int Lq = p.Lq, Lk = p.Lk, A = p.A, R = 2 * A;
  const bool p2c = (p.flags & 2) != 0;
  BT* cbs = reinterpret_cast<BT*>(uni);
  BT* pbw = reinterpret_cast<BT*>(uni) + CB_ELEMS + w * PB_ELEMS;
  T* dsd_all = reinterpret_cast<T*>(uni);
  T* dsd = dsd_all + w * XW * DS2;
  T* Ap = reinterpret_cast<T*>(uni + DSD_BYTES);
  const float sl2 = p.scale * kLog2e;
  const int KT = (Lk + BKW - 1) / BKW;
  const int nqt = (Lq + BQ - 1) / BQ;

  f32x4 dqra[OWN][ND];
#pragma unroll
  for (int k = 0; k < OWN; ++k)
#pragma unroll
    for (int db = 0; db < ND; ++db) dqra[k][db] = zero4();
  int cur_h = -1, slot = 0;
  const int it0 = item_begin(blockIdx.x, plan.items, plan.grid);
  const int it1 = item_begin(blockIdx.x + 1, plan.items, plan.grid);

  for (int item = it0; item < it1; ++item) {
    const int h = item / plan.per_head;
    const int b = (item % plan.per_head) / KT;
    const int kt = item % KT;
    if (h != cur_h) {
      if (cur_h >= 0 && p2c) {
        store_partial<D>(part + ((int64_t)blockIdx.x * plan.slots + slot) * plan.prow * D, plan.prow, dqra, p.scale,
                         w, g, c16);
        ++slot;
      }
#pragma unroll
      for (int k = 0; k < OWN; ++k)
#pragma unroll
        for (int db = 0; db < ND; ++db) dqra[k][db] = zero4();
      cur_h = h;
    }
    const int j0 = kt * BKW;
    const int jw = j0 + w * WK;
    const T* qbase = (const T*)p.q + (int64_t)b * p.qs[0] + (int64_t)h * p.qs[2];
    const T* kbase = (const T*)p.k + (int64_t)b * p.ks[0] + (int64_t)h * p.ks[2];
    const T* vbase = (const T*)p.v + (int64_t)b * p.vs[0] + (int64_t)h * p.vs[2];
    const T* dobase = (const T*)bp.dout + (int64_t)b * bp.dos[0] + (int64_t)h * bp.dos[2];
    const T* krh = (p.flags & 1) ? (const T*)p.kr + (int64_t)h * p.krs[0] : nullptr;
    const T* qrh = p2c ? (const T*)p.qr + (int64_t)h * p.qrs[0] : nullptr;
    const uint8_t* kkb = (MASK == MASK_KEY) ? p.kk + (int64_t)b * p.kkb : nullptr;
    const uint8_t* pkb = (MASK == MASK_PAIR) ? p.pk + (int64_t)b * p.pkb : nullptr;
    const float* lseb = p.lse + ((int64_t)b * p.H + h) * Lq;
    const float* dltb = bp.delta + ((int64_t)b * p.H + h) * Lq;

    int jcol[2];
    bool jkeep[2];
    frag kb[2][NS], vb[2][NS];
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) {
      const int j = jw + 16 * jb + c16;
      jcol[jb] = j;
      const bool valid = j < Lk;
      jkeep[jb] = valid && (MASK != MASK_KEY || kkb[j] != 0);
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        kb[jb][s] = valid ? M::load_contig(kbase + (int64_t)j * p.ks[1], s, g) : M::zero();
        vb[jb][s] = valid ? M::load_contig(vbase + (int64_t)j * p.vs[1], s, g) : M::zero();
      }
    }

    __syncthreads();  // previous item's LDS use is over
    if constexpr (BF) {
      if (p2c) load_rows<T, D, BKW, 256>(Ks, KSTR, nullptr, 0, kbase, p.ks[1], j0, Lk, tid);
    }
    int wg_keep = 0;
    if (tid < BKW) {
      const int j = j0 + tid;
      if (j < Lk) wg_keep = (MASK == MASK_KEY) ? kkb[j] != 0 : 1;
    }
    const bool any_key = __syncthreads_or(wg_keep);

    f32x4 dka[ND][2], dva[ND][2];
#pragma unroll
    for (int db = 0; db < ND; ++db) dka[db][0] = dka[db][1] = dva[db][0] = dva[db][1] = zero4();

    for (int qi = 0; any_key && qi < nqt; ++qi) {
      const int i0 = qi * BQ;
      if (MASK == MASK_KEY) {
        int live = 0;
        if (tid < BQ) live = (i0 + tid < Lq) && kkb[i0 + tid];
        if (!__syncthreads_or(live)) continue;
      } else if (MASK == MASK_PAIR) {
        int keep = 0;
        const int r = tid >> 2, quarter = tid & 3;
        const int i = i0 + r;
        if (i < Lq && pkb[(int64_t)i * p.pkq + i]) {
          const uint8_t* row = pkb + (int64_t)i * p.pkq;
          const int jb0 = j0 + quarter * (BKW / 4);
          const int jend = min(jb0 + BKW / 4, Lk);
          for (int j = jb0; j < jend; ++j) keep |= row[j];
        }
        if (!__syncthreads_or(keep)) continue;
      }
      __syncthreads();
      load_rows<T, D, BQ, 256>(Qs, KSTR, nullptr, 0, qbase, p.qs[1], i0, Lq, tid);
      load_rows<T, D, BQ, 256>(dOs, KSTR, nullptr, 0, dobase, bp.dos[1], i0, Lq, tid);
      if (tid < BQ) {
        const int i = i0 + tid;
        bool live = i < Lq;
        if (MASK == MASK_KEY && live) live = kkb[i] != 0;
        if (MASK == MASK_PAIR && live) live = pkb[(int64_t)i * p.pkq + i] != 0;
        rowv[tid] = live ? lseb[i] * kLog2e : INFINITY;
        rowv[BQ + tid] = (i < Lq) ? dltb[i] : 0.f;
      }
      const int dbase = i0 - j0 - (BKW - 1);
      if (p.flags) load_row_tables_at(crow, prow, p.rel, dbase, Lq, Lk, A, tid);
      // Window of Qr rows [p(x=191), p(x=0)] for the p2c band and the dK product.
      int wide = 0;
      int plo0 = 0;
      if (p2c) {
        plo0 = p2c_row(min(max(p.rel[min(max(dbase + XG - 1, -(Lk - 1)), Lq - 1) + Lk - 1], -A), A), A);
        const int phi0 = p2c_row(min(max(p.rel[min(max(dbase, -(Lk - 1)), Lq - 1) + Lk - 1], -A), A), A);
        wide = (phi0 - plo0 + 1 > ARN) ? 1 : 0;
        if (!wide) stage_rows_window<T, D, ARN>(QrW, KSTR, qrh, p.qrs[1], plo0, phi0, R, tid);
      }
      const bool fast = !__syncthreads_or(wide);

      // ---- scores (queries down, keys across) -------------------------------------------
      frag qa[4][NS];
#pragma unroll
      for (int ib = 0; ib < 4; ++ib)
#pragma unroll
        for (int s = 0; s < NS; ++s) qa[ib][s] = M::load_contig(&Qs[(16 * ib + c16) * KSTR], s, g);
      f32x4 sc[2][4];
#pragma unroll
      for (int ib = 0; ib < 4; ++ib)
#pragma unroll
        for (int jb = 0; jb < 2; ++jb) {
          f32x4 acc = zero4();
#pragma unroll
          for (int s = 0; s < NS; ++s) acc = M::mma(qa[ib][s], kb[jb][s], acc);
          sc[jb][ib] = acc * sl2;
        }
      if (p.flags)
        add_delta_bands_S<T, D>(sc, qa, kb, cbs, pbw, crow, prow, w, g, c16, krh, p.krs[1], qrh, p.qrs[1], p.flags,
                                sl2, (p2c && fast) ? (const T*)QrW : nullptr, KSTR, plo0);

      // ---- P, dP, dS ----------------------------------------------------------------------
      f32x4 pp[2][4], ds[2][4];
#pragma unroll
      for (int ib = 0; ib < 4; ++ib) {
        frag dof[NS];
#pragma unroll
        for (int s = 0; s < NS; ++s) dof[s] = M::load_contig(&dOs[(16 * ib + c16) * KSTR], s, g);
#pragma unroll
        for (int jb = 0; jb < 2; ++jb) {
          f32x4 dp = zero4();
#pragma unroll
          for (int s = 0; s < NS; ++s) dp = M::mma(dof[s], vb[jb][s], dp);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int il = 16 * ib + 4 * g + e;
            const int i = i0 + il;
            bool keep = jkeep[jb];
            if (MASK == MASK_PAIR) keep = keep && i < Lq && pkb[(int64_t)i * p.pkq + jcol[jb]] != 0;
            const float pe = keep ? exp2f(sc[jb][ib][e] - rowv[il]) : 0.f;
            pp[jb][ib][e] = pe;
            ds[jb][ib][e] = pe * (dp[e] - rowv[BQ + il]);
          }
        }
      }

      // ---- dV^T += dO^T P,  dK^T += Q^T dS (dO^T, Q^T read transposed) -----------------------
#pragma unroll
      for (int s = 0; s < BQ / M::KSTEP; ++s) {
        frag pf[2], df[2];
#pragma unroll
        for (int jb = 0; jb < 2; ++jb) {
          pf[jb] = M::from_acc(pp[jb], s);
          df[jb] = M::from_acc(ds[jb], s);
        }
#pragma unroll
        for (int db = 0; db < ND; ++db) {
          const frag dotf = tr_acc<T>(dOs, KSTR, s * M::KSTEP, 16 * db, g, c16);
          const frag qtf = tr_acc<T>(Qs, KSTR, s * M::KSTEP, 16 * db, g, c16);
#pragma unroll
          for (int jb = 0; jb < 2; ++jb) {
            dva[db][jb] = M::mma(dotf, pf[jb], dva[db][jb]);
            dka[db][jb] = M::mma(qtf, df[jb], dka[db][jb]);
          }
        }
      }

      // ---- p2c gradients --------------------------------------------------------------------
      if (p2c) {
        const int plo = prow[XG - 1];                // p(x) is non-increasing in x
        const int np = prow[0] - plo + 1;
        __syncthreads();  // score bands are consumed; the union region is free
        {
          constexpr int DSD_V = XW * DS2 * (int)sizeof(T) / 16;
          f32x4* z = reinterpret_cast<f32x4*>(dsd);
          for (int x = (tid & 63); x < DSD_V; x += 64) z[x] = zero4();
          wave_lds_sync();
          // x_local = (16*ib + 4*g + e) - (16*jb + c16) + 31, column j_local = 16*jb + c16
          T* base = dsd + (4 * g - c16 + 31) * DS2 + c16;
#pragma unroll
          for (int jb = 0; jb < 2; ++jb)
#pragma unroll
            for (int ib = 0; ib < 4; ++ib)
#pragma unroll
              for (int e = 0; e < 4; ++e) base[(16 * ib + e - 16 * jb) * DS2 + 16 * jb] = (T)ds[jb][ib][e];
        }
        for (int cb = plo; cb < plo + np; cb += ARN) {
          const int ncr = min(ARN, plo + np - cb);
          if (!fast) {
            __syncthreads();
            stage_rows_window<T, D, ARN>(QrW, KSTR, qrh, p.qrs[1], cb, cb + ncr - 1, R, tid);
          }
          if (tid < ARN) {
            const int r = cb + tid;
            int lo = 0, hi = XG;
            while (lo < hi) {  // first x with prow[x] <= r
              const int mid = (lo + hi) >> 1;
              if (prow[mid] > r) lo = mid + 1; else hi = mid;
            }
            int lo2 = lo, hi2 = XG;
            while (lo2 < hi2) {  // first x with prow[x] < r
              const int mid = (lo2 + hi2) >> 1;
              if (prow[mid] >= r) lo2 = mid + 1; else hi2 = mid;
            }
            xlo[tid] = (short)lo;
            xhi[tid] = (short)(lo2 - 1);
          }
          __syncthreads();
          // fold: Ap[p][j] = sum_{x in X(p)} dSd[x][j]
          for (int q = tid; q < ARN * (BKW / 8); q += 256) {
            const int rr = q >> 4, c = q & 15;
            const int ws = c >> 2, jl = 8 * c - WK * ws;
            float acc[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[e] = 0.f;
            if (rr < ncr) {
              const int x1 = xhi[rr];
              for (int x = xlo[rr]; x <= x1; ++x) {
                const int xl = x - (XW - WK * ws);
                if (xl >= 0 && xl < XW) {
                  const T* src = dsd_all + (ws * XW + xl) * DS2 + jl;
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
            T* dst = Ap + rr * AR_STR + 8 * c;
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
          // dK^T[d][j] += sum_p QrW^T[d][p] Ap[p][j]   (this wave's 32 keys)
          const int nsteps = (ncr + M::KSTEP - 1) / M::KSTEP;
          for (int s = 0; s < nsteps; ++s) {
            frag bfr[2];
#pragma unroll
            for (int jb = 0; jb < 2; ++jb) bfr[jb] = tr_contig<T>(Ap, AR_STR, s * M::KSTEP, WK * w + 16 * jb, g, c16);
#pragma unroll
            for (int db = 0; db < ND; ++db) {
              const frag af = tr_contig<T>(QrW, KSTR, s * M::KSTEP, 16 * db, g, c16);
#pragma unroll
              for (int jb = 0; jb < 2; ++jb) dka[db][jb] = M::mma(af, bfr[jb], dka[db][jb]);
            }
          }
          // dQr[p][d] += sum_j Ap[p][j] K[j][d]   (16-row blocks this wave owns)
          const int blo = cb >> 4, bhi = (cb + ncr - 1) >> 4;
          for (int rb = blo + ((w - blo % NW) + NW) % NW; rb <= bhi; rb += NW) {
            const int rr = 16 * rb + c16 - cb;
            const bool rok = rr >= 0 && rr < ncr;
            f32x4 res[ND];
#pragma unroll
            for (int db = 0; db < ND; ++db) res[db] = zero4();
#pragma unroll
            for (int s = 0; s < BKW / M::KSTEP; ++s) {
              const frag af = rok ? M::load_contig(Ap + rr * AR_STR, s, g) : M::zero();
#pragma unroll
              for (int db = 0; db < ND; ++db) {
                frag bk;
                if constexpr (BF) {
                  bk = tr_contig<T>(Ks, KSTR, s * M::KSTEP, 16 * db, g, c16);
                } else {
#pragma unroll
                  for (int e = 0; e < 4; ++e) {
                    const int j = j0 + s * M::KSTEP + 4 * g + e;
                    bk[e] = (j < Lk) ? kbase[(int64_t)j * p.ks[1] + 16 * db + c16] : 0.f;
                  }
                }
                res[db] = M::mma(af, bk, res[db]);
              }
            }
            const int k = rb / NW;
            bool held = false;
#pragma unroll
            for (int kk = 0; kk < OWN; ++kk) {
              if (k == kk) {
#pragma unroll
                for (int db = 0; db < ND; ++db) dqra[kk][db] += res[db];
                held = true;
              }
            }
            if (!held) {
#pragma unroll
              for (int db = 0; db < ND; ++db) res[db] *= p.scale;
              atomic_rows<D>(bp.dqr + (int64_t)h * R * D, R, 16 * rb, res, g, c16);
            }
          }
        }
      }
    }

    // ---- dK, dV of the item ----------------------------------------------------------------
    T* dkbase = (T*)bp.dk + (int64_t)b * bp.dks[0] + (int64_t)h * bp.dks[2];
    T* dvbase = (T*)bp.dv + (int64_t)b * bp.dvs[0] + (int64_t)h * bp.dvs[2];
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) {
      const int j = jcol[jb];
      if (j < Lk) {
        T* krow = dkbase + (int64_t)j * bp.dks[1];
        T* vrow = dvbase + (int64_t)j * bp.dvs[1];
#pragma unroll
        for (int db = 0; db < ND; ++db) {
          typedef T vec4 __attribute__((ext_vector_type(4)));
          vec4 kv, vv;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            kv[e] = (T)(dka[db][jb][e] * p.scale);
            vv[e] = (T)(dva[db][jb][e]);
          }
          *reinterpret_cast<vec4*>(krow + 16 * db + 4 * g) = kv;
          *reinterpret_cast<vec4*>(vrow + 16 * db + 4 * g) = vv;
        }
      }
    }
  }
  if (cur_h >= 0 && p2c) {
    store_partial<D>(part + ((int64_t)blockIdx.x * plan.slots + slot) * plan.prow * D, plan.prow, dqra, p.scale, w, g,
                     c16);
  }
}

}  // namespace dsa
