// dsa_bwd_dkdv.h — dK, dV and dS^T of the fused disentangled attention
// (gfx950).
//
// One workgroup = 4 waves = one (batch b, head h, 128-key tile); wave w owns
// keys [j0 + 32w, j0 + 32w + 32) and streams 64-query tiles:
//   scores        y = (Q K^T + c2p + p2c) * scale*log2e, queries down / keys
//                 across: the c2p band (the queries are shared by the
//                 waves) is computed once per workgroup, the p2c band per wave
//   P, dP, dS     P = exp2(y - lse*log2e), dP = dO V^T, dS = P (dP - Delta)
//   dV^T         += dO^T P,  dK^T += Q^T dS        (dO^T, Q^T read transposed
//                                                   from LDS)
//   dS^T          stored to the workspace (row j, 4 consecutive queries per
//                 lane): the dq, dkp and table kernels read it
// With p2c, dK is left unscaled in fp32 in the workspace and completed by
// dsa_bwd_dkp_kernel (dsa_bwd_dkp.h), which adds the p2c term from dS^T.
// Every query tile of the padded extent is visited, so dS^T is fully written
// (zeros for masked pairs, dead rows and padding).
#pragma once

#include "dsa_bwd.h"

namespace dsa {

namespace kvcfg {
constexpr int NW = 4, WK = 32, BKW = 128, BQ = 64;
constexpr int XW = 96;            // offset rows per wave (95 used)
constexpr int XG = 192;           // offset rows per workgroup (191 used)
constexpr int CBS = XG + 5;       // shared c2p band row stride [i][x]
constexpr int PBS = WK + 1;       // per-wave p2c band row stride [x][j]
constexpr int CB_ELEMS = BQ * CBS;
constexpr int PB_ELEMS = XW * PBS;
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
//   cbs: shared c2p band (BQ * CBS), pbw: this wave's p2c band (XW * PBS),
//   both unscaled; sl2 is applied as the band values are added
// Contains one __syncthreads.
template <typename T, int D>
DSA_DEV void add_delta_bands_S(f32x4 (&y)[2][4], const typename Mfma<T>::frag (&qa)[4][D / Mfma<T>::KSTEP],
                               const typename Mfma<T>::frag (&kb)[2][D / Mfma<T>::KSTEP],
                               typename BandType<T>::type* cbs, typename BandType<T>::type* pbw, const short* crow,
                               const short* prow, int w, int g, int c16, const T* krh, int64_t krs, const T* qrh,
                               int64_t qrs, int flags, float sl2) {
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
        store_band4<BT>(cbs + (16 * ib + 4 * g) * CBS + 16 * xb + c16, CBS, acc);
      }
    }
  }
  if (flags & 2) {  // per-wave p2c band: PB[x][j] = Qr[p(x)] . k_j, x over the wave's window
    const int xw0 = XW - WK * w;
#pragma unroll
    for (int xb = 0; xb < XW / 16; ++xb) {
      const int row = prow[min(xw0 + 16 * xb + c16, XG - 1)];
      frag af[NS];
#pragma unroll
      for (int s = 0; s < NS; ++s) af[s] = M::load_contig(qrh + (int64_t)row * qrs, s, g);
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) {
        f32x4 acc = zero4();
#pragma unroll
        for (int s = 0; s < NS; ++s) acc = M::mma(af[s], kb[jb][s], acc);
        store_band4<BT>(pbw + (16 * xb + 4 * g) * PBS + 16 * jb + c16, PBS, acc);
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
        for (int e = 0; e < 4; ++e)
          y[jb][ib][e] = __builtin_fmaf((float)base[(16 * ib + e) * CBS + 16 * ib + e - 16 * jb], sl2, y[jb][ib][e]);
  }
  if (flags & 2) {
    // x_local = (16*ib + 4*g + e) - (16*jb + c16) + 31, column j_local = 16*jb + c16
    const BT* base = pbw + (4 * g - c16 + 31) * PBS + c16;
#pragma unroll
    for (int jb = 0; jb < 2; ++jb)
#pragma unroll
      for (int ib = 0; ib < 4; ++ib)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          y[jb][ib][e] = __builtin_fmaf((float)base[(16 * ib + e - 16 * jb) * PBS + 16 * jb], sl2, y[jb][ib][e]);
  }
}

// Stores a lane's 2 x 4 C tiles of dS (query rows 16*ib + 4*g + e, key
// column 16*jb + c16 of the wave) as dS^T rows: 4 consecutive queries per
// store.  With zero = true, stores zeros.
template <typename T>
DSA_DEV void store_dst(T* dst_wave, int LqP, int i0, const f32x4 (&ds)[2][4], bool zero, int g, int c16) {
  typedef T vec4 __attribute__((ext_vector_type(4)));
#pragma unroll
  for (int jb = 0; jb < 2; ++jb) {
    T* row = dst_wave + (int64_t)(16 * jb + c16) * LqP + i0 + 4 * g;
#pragma unroll
    for (int ib = 0; ib < 4; ++ib) {
      vec4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = zero ? (T)0.0f : (T)ds[jb][ib][e];
      *reinterpret_cast<vec4*>(row + 16 * ib) = v;
    }
  }
}

template <typename T, int D, int MASK>
__global__ __launch_bounds__(256, sizeof(T) == 2 ? 2 : 1) void dsa_bwd_dkdv_kernel(BwdParams bp) {
  using namespace kvcfg;
  using M = Mfma<T>;
  typedef typename M::frag frag;
  typedef typename BandType<T>::type BT;
  constexpr int NS = D / M::KSTEP;
  constexpr int ND = D / 16;
  constexpr int KSTR = D + Pad<T>::v;
  constexpr int UNI_BYTES = (CB_ELEMS + NW * PB_ELEMS) * (int)sizeof(BT);
  const FwdParams& p = bp.f;

  __shared__ __align__(16) T Qs[BQ * KSTR];
  __shared__ __align__(16) T dOs[BQ * KSTR];
  __shared__ float rowv[2 * BQ];
  __shared__ short crow[XG], prow[XG];
  __shared__ __align__(16) char uni[UNI_BYTES];

  const int tid = threadIdx.x;
  const int w = tid >> 6, g = (tid & 63) >> 4, c16 = tid & 15;
  const int Lq = p.Lq, Lk = p.Lk, A = p.A;
  const int kt = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const bool p2c = (p.flags & 2) != 0;
  BT* cbs = reinterpret_cast<BT*>(uni);
  BT* pbw = reinterpret_cast<BT*>(uni) + CB_ELEMS + w * PB_ELEMS;
  const float sl2 = p.scale * kLog2e;
  const int nqt = bp.LqP / BQ;

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
  T* dstw = (T*)bp.dst + ((int64_t)(b * p.H + h) * bp.LkP + jw) * bp.LqP;

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

  int wg_keep = 0;
  if (tid < BKW) {
    const int j = j0 + tid;
    if (j < Lk) wg_keep = (MASK == MASK_KEY) ? kkb[j] != 0 : 1;
  }
  const bool any_key = __syncthreads_or(wg_keep);

  f32x4 dka[ND][2], dva[ND][2];
#pragma unroll
  for (int db = 0; db < ND; ++db) dka[db][0] = dka[db][1] = dva[db][0] = dva[db][1] = zero4();
  const f32x4 zt[2][4] = {};

  for (int qi = 0; qi < nqt; ++qi) {
    const int i0 = qi * BQ;
    // Tiles without a kept (query, key) pair store zeros and are skipped.
    bool skip = !any_key || i0 >= Lq;
    if (!skip && MASK == MASK_KEY) {
      int live = 0;
      if (tid < BQ) live = (i0 + tid < Lq) && kkb[i0 + tid];
      skip = !__syncthreads_or(live);
    } else if (!skip && MASK == MASK_PAIR) {
      int keep = 0;
      const int r = tid >> 2, quarter = tid & 3;
      const int i = i0 + r;
      if (i < Lq && pkb[(int64_t)i * p.pkq + i]) {
        const uint8_t* row = pkb + (int64_t)i * p.pkq;
        const int jb0 = j0 + quarter * (BKW / 4);
        const int jend = min(jb0 + BKW / 4, Lk);
        for (int j = jb0; j < jend; ++j) keep |= row[j];
      }
      skip = !__syncthreads_or(keep);
    }
    if (skip) {
      store_dst<T>(dstw, bp.LqP, i0, zt, true, g, c16);
      continue;
    }
    __syncthreads();  // previous tile's LDS readers are done
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
    if (p.flags) load_row_tables_at(crow, prow, p.rel, i0 - j0 - (BKW - 1), Lq, Lk, A, tid);
    __syncthreads();

    // ---- scores (queries down, keys across) -------------------------------------------
    f32x4 sc[2][4];
    {
      frag qa[4][NS];
#pragma unroll
      for (int ib = 0; ib < 4; ++ib)
#pragma unroll
        for (int s = 0; s < NS; ++s) qa[ib][s] = M::load_contig(&Qs[(16 * ib + c16) * KSTR], s, g);
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
                                sl2);
    }

    // ---- per 32-query half: P, dP, dS, then dV^T += dO^T P, dK^T += Q^T dS ---------------
    // (dO^T, Q^T read transposed from LDS); dS is also stored to dS^T.
    constexpr int HALVES = 2, IBH = 4 / HALVES, SPH = IBH * 16 / M::KSTEP;
#pragma unroll
    for (int hh = 0; hh < HALVES; ++hh) {
      f32x4 pp[2][IBH], dsh[2][IBH];
#pragma unroll
      for (int t = 0; t < IBH; ++t) {
        const int ib = IBH * hh + t;
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
            const float pe = keep ? __builtin_amdgcn_exp2f(sc[jb][ib][e] - rowv[il]) : 0.f;
            pp[jb][t][e] = pe;
            dsh[jb][t][e] = pe * (dp[e] - rowv[BQ + il]);
          }
        }
      }
      // dS^T rows: 4 consecutive queries per store
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) {
        typedef T vec4 __attribute__((ext_vector_type(4)));
        T* row = dstw + (int64_t)(16 * jb + c16) * bp.LqP + i0 + 4 * g;
#pragma unroll
        for (int t = 0; t < IBH; ++t) {
          vec4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = (T)dsh[jb][t][e];
          *reinterpret_cast<vec4*>(row + 16 * (IBH * hh + t)) = v;
        }
      }
#pragma unroll
      for (int sh = 0; sh < SPH; ++sh) {
        const int s = hh * SPH + sh;
        frag pf[2], df[2];
#pragma unroll
        for (int jb = 0; jb < 2; ++jb) {
          pf[jb] = M::from_acc(pp[jb], sh);
          df[jb] = M::from_acc(dsh[jb], sh);
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
    }
  }

  // ---- dK, dV ------------------------------------------------------------------------------
  T* dkbase = (T*)bp.dk + (int64_t)b * bp.dks[0] + (int64_t)h * bp.dks[2];
  T* dvbase = (T*)bp.dv + (int64_t)b * bp.dvs[0] + (int64_t)h * bp.dvs[2];
  float* dkcw = p2c ? bp.dkc + ((int64_t)(b * p.H + h) * bp.LkP) * D : nullptr;
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
        if (p2c) {  // content part of dK, completed by dsa_bwd_dkp_kernel
          *reinterpret_cast<f32x4*>(dkcw + (int64_t)j * D + 16 * db + 4 * g) = dka[db][jb];
        } else {
          *reinterpret_cast<vec4*>(krow + 16 * db + 4 * g) = kv;
        }
        *reinterpret_cast<vec4*>(vrow + 16 * db + 4 * g) = vv;
      }
    }
  }
}

}  // namespace dsa
