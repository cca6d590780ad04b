// dsa_bwd.h — backward of the fused disentangled attention (gfx950).
//
// With s = scale, P the softmax probabilities (recomputed from the saved
// logsumexp), Delta_i = dO_i . O_i and dS = P * (dP - Delta):
//   dP = dO V^T
//   dV = P^T dO
//   dQ = s dS K          + s sum_j dS_ij Kr[c(i-j)]
//   dK = s dS^T Q        + s sum_i dS_ij Qr[p(i-j)]
//   dKr[r] = s sum_{b,i,j: c(i-j)=r} dS_ij q_i
//   dQr[r] = s sum_{b,i,j: p(i-j)=r} dS_ij k_j
// (ATen autograd of deberta_v2_native.py:592-652 with the c2p/p2c gathers of
// :389-410; masked keys and dead query rows have P = 0 and so dS = 0.)
//
// Two kernels share the score recompute:
//   dsa_bwd_dq_kernel   one (b, h, 128-query tile) per workgroup, loops over
//                       64-key tiles; produces dQ and dKr.
//   dsa_bwd_dkdv_kernel one (b, h, 128-key tile) per workgroup, loops over
//                       64-query tiles; produces dK, dV and dQr.
// The relative-table gradients are bucket scatters of dS: per tile, dS is
// scatter-added (LDS float atomics) into a band indexed by table row, which
// is then contracted with Q (dKr) or K (dQr) on MFMA.  Each wave owns every
// fourth 16-row block of the table and keeps its blocks' partial sums in
// registers for the whole loop (8 blocks = 128 rows per wave, 512 rows per
// workgroup); they are added to the fp32 output once, at the end.
#pragma once

#include "dsa_tiles.h"

namespace dsa {

namespace bwdcfg {
constexpr int NW = 4;
constexpr int TILE_OWN = 128;  // rows owned by a workgroup (queries for dq, keys for dkdv)
constexpr int TILE_LOOP = 64;  // rows per loop step
constexpr int WB = 192;        // workgroup band rows per chunk (>= 128 + 64 - 1)
constexpr int WB_STR = 132;    // workgroup band row stride (floats, 16-byte rows)
constexpr int SCR = 64 * (tilecfg::BAND + 1);
constexpr int UNION = (NW * SCR > WB * WB_STR) ? NW * SCR : WB * WB_STR;
constexpr int OWN_SLOTS = 8;   // register-held 16-row blocks per wave
constexpr int TBL = TILE_OWN + TILE_LOOP;
}  // namespace bwdcfg

// Adds a 16 x D block (rows r0.., C layout: col d = 16*db + c16, rows 4g+e)
// to an fp32 [R, D] table with device-scope atomics.
template <int D>
DSA_DEV void atomic_add_block(float* tab, int R, int r0, const f32x4 (&v)[D / 16], int g, int c16) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int r = r0 + 4 * g + e;
    if (r < R) {
#pragma unroll
      for (int db = 0; db < D / 16; ++db) atomicAdd(tab + (int64_t)r * D + 16 * db + c16, v[db][e]);
    }
  }
}

// Loads a B fragment whose k index runs down a column of a row-major LDS
// array: element (k, col) at base[k * str + col].  k-set CONTIG for bf16.
template <typename T>
DSA_DEV typename Mfma<T>::frag load_col_contig(const T* base, int str, int col, int k0, int g) {
  using M = Mfma<T>;
  typename M::frag f;
  if constexpr (sizeof(T) == 2) {
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = base[(k0 + 8 * g + e) * str + col];
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) f[e] = base[(k0 + 4 * g + e) * str + col];
  }
  return f;
}

// Same with the ACC k-set.
template <typename T>
DSA_DEV typename Mfma<T>::frag load_col_acc(const T* base, int str, int col, int k0, int g) {
  using M = Mfma<T>;
  typename M::frag f;
#pragma unroll
  for (int e = 0; e < M::FRAG_ELEMS; ++e) f[e] = base[(k0 + M::acc_k(g, e)) * str + col];
  return f;
}

// fp32 band rows -> fragment (CONTIG k-set), rows outside [0, nrow) read 0.
template <typename T>
DSA_DEV typename Mfma<T>::frag band_row_frag(const float* band, int row, int nrow, int k0, int g) {
  using M = Mfma<T>;
  float v[8];
  const bool ok = row >= 0 && row < nrow;
  if constexpr (sizeof(T) == 2) {
    const float* src = band + row * bwdcfg::WB_STR + k0 + 8 * g;
    f32x4 a = ok ? *reinterpret_cast<const f32x4*>(src) : zero4();
    f32x4 b2 = ok ? *reinterpret_cast<const f32x4*>(src + 4) : zero4();
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = a[e];
      v[4 + e] = b2[e];
    }
    typename M::frag f;
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = (bf16)v[e];
    return f;
  } else {
    const float* src = band + row * bwdcfg::WB_STR + k0 + 4 * g;
    return ok ? *reinterpret_cast<const f32x4*>(src) : zero4();
  }
}

// fp32 band column -> fragment (CONTIG k-set over band rows), rows outside
// [lo, hi] (band-relative) read 0.
template <typename T>
DSA_DEV typename Mfma<T>::frag band_col_frag(const float* band, int col, int k0, int lo, int hi, int g) {
  using M = Mfma<T>;
  typename M::frag f;
  if constexpr (sizeof(T) == 2) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int r = k0 + 8 * g + e;
      f[e] = (bf16)((r >= lo && r <= hi) ? band[r * bwdcfg::WB_STR + col] : 0.f);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int r = k0 + 4 * g + e;
      f[e] = (r >= lo && r <= hi) ? band[r * bwdcfg::WB_STR + col] : 0.f;
    }
  }
  return f;
}

// ===========================================================================
// dK / dV / dQr kernel
// ===========================================================================
template <typename T, int D, int MASK>
__global__ __launch_bounds__(256, 1) void dsa_bwd_dkdv_kernel(BwdParams bp) {
  using namespace bwdcfg;
  using M = Mfma<T>;
  typedef typename M::frag frag;
  constexpr int NS = D / M::KSTEP;
  constexpr int ND = D / 16;
  constexpr int BKW = TILE_OWN, BQ = TILE_LOOP, WK = 32;
  constexpr bool BF = sizeof(T) == 2;
  constexpr int QSTR = D + Pad<T>::v;
  constexpr int TSTR = BQ + Pad<T>::v;    // Qt / dOt: [D][BQ]
  constexpr int KTSTR = BKW + Pad<T>::v;  // Kt: [D][BKW]
  const FwdParams& p = bp.f;

  __shared__ __align__(16) T Qs[BQ * QSTR];
  __shared__ __align__(16) T dOs[BQ * QSTR];
  __shared__ __align__(16) T Qt[BF ? D * TSTR : 1];
  __shared__ __align__(16) T dOt[BF ? D * TSTR : 1];
  __shared__ __align__(16) T Kt[BF ? D * KTSTR : 1];
  __shared__ float rowv[2 * BQ];  // lse2, delta for the query tile
  __shared__ short tbl[TBL];
  __shared__ __align__(16) float uni[UNION];

  const int tid = threadIdx.x;
  const int w = tid >> 6, l = tid & 63, g = l >> 4, c16 = l & 15;
  const int kt = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int Lq = p.Lq, Lk = p.Lk, A = p.A, R = 2 * A;
  const int j0 = kt * BKW;
  const int jw = j0 + w * WK;
  float* scr = uni + w * SCR;
  float* band = uni;

  const T* qbase = (const T*)p.q + (int64_t)b * p.qs[0] + (int64_t)h * p.qs[2];
  const T* kbase = (const T*)p.k + (int64_t)b * p.ks[0] + (int64_t)h * p.ks[2];
  const T* vbase = (const T*)p.v + (int64_t)b * p.vs[0] + (int64_t)h * p.vs[2];
  const T* dobase = (const T*)bp.dout + (int64_t)b * bp.dos[0] + (int64_t)h * bp.dos[2];
  const T* krh = (p.flags & 1) ? (const T*)p.kr + (int64_t)h * p.krs[0] : nullptr;
  const T* qrh = (p.flags & 2) ? (const T*)p.qr + (int64_t)h * p.qrs[0] : nullptr;
  const T* qrTh = (p.flags & 2) ? (const T*)bp.qrT + (int64_t)h * D * bp.Rpad : nullptr;
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
  if constexpr (BF) {
    if (p.flags & 2) load_rows<T, D, BKW, 256>(nullptr, 0, Kt, KTSTR, kbase, p.ks[1], j0, Lk, tid);
  }

  f32x4 dka[ND][2], dva[ND][2];
#pragma unroll
  for (int db = 0; db < ND; ++db) dka[db][0] = dka[db][1] = dva[db][0] = dva[db][1] = zero4();
  f32x4 dqra[OWN_SLOTS][ND];
#pragma unroll
  for (int k = 0; k < OWN_SLOTS; ++k)
#pragma unroll
    for (int db = 0; db < ND; ++db) dqra[k][db] = zero4();
  uint32_t touched = 0;

  const float sl2 = p.scale * kLog2e;
  const int nqt = (Lq + BQ - 1) / BQ;

  // Keys this workgroup holds that any query could keep.
  int wg_keep = 0;
  if (tid < BKW) {
    const int j = j0 + tid;
    if (j < Lk) wg_keep = (MASK == MASK_KEY) ? kkb[j] != 0 : 1;
  }
  const bool any_key = __syncthreads_or(wg_keep);

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
    load_rows<T, D, BQ, 256>(Qs, QSTR, BF ? Qt : nullptr, TSTR, qbase, p.qs[1], i0, Lq, tid);
    load_rows<T, D, BQ, 256>(dOs, QSTR, BF ? dOt : nullptr, TSTR, dobase, bp.dos[1], i0, Lq, tid);
    if (tid < BQ) {
      const int i = i0 + tid;
      bool live = i < Lq;
      if (MASK == MASK_KEY && live) live = kkb[i] != 0;
      if (MASK == MASK_PAIR && live) live = pkb[(int64_t)i * p.pkq + i] != 0;
      rowv[tid] = live ? lseb[i] * kLog2e : INFINITY;
      rowv[BQ + tid] = (i < Lq) ? dltb[i] : 0.f;
    }
    if (p.flags) load_rel_window(tbl, p.rel, i0 - j0 - (BKW - 1), BQ + BKW - 1, Lq, Lk, A, tid, 256);
    __syncthreads();

    // ---- recompute scores (queries down, keys across) -----------------------------
    frag qa[4][NS];
#pragma unroll
    for (int ib = 0; ib < 4; ++ib)
#pragma unroll
      for (int s = 0; s < NS; ++s) qa[ib][s] = M::load_contig(&Qs[(16 * ib + c16) * QSTR], s, g);
    f32x4 sc[2][4];
    score_tile_S<T, D>(sc, qa, kb, scr, tbl, (BKW - 1) - w * WK, l, g, c16, krh, p.krs[1], qrh, p.qrs[1], A,
                       p.flags);

    // ---- P, dP, dS ---------------------------------------------------------------------
    f32x4 pp[2][4], ds[2][4];
#pragma unroll
    for (int ib = 0; ib < 4; ++ib) {
      frag dof[NS];
#pragma unroll
      for (int s = 0; s < NS; ++s) dof[s] = M::load_contig(&dOs[(16 * ib + c16) * QSTR], s, g);
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
          const float pe = keep ? exp2f(sc[jb][ib][e] * sl2 - rowv[il]) : 0.f;
          pp[jb][ib][e] = pe;
          ds[jb][ib][e] = pe * (dp[e] - rowv[BQ + il]);
        }
      }
    }

    // ---- dV^T += dO^T P,  dK^T += Q^T dS ------------------------------------------------
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
        frag dof, qtf;
        if constexpr (BF) {
          dof = M::load_acc(&dOt[(16 * db + c16) * TSTR], s, g);
          qtf = M::load_acc(&Qt[(16 * db + c16) * TSTR], s, g);
        } else {
          dof = load_col_acc<T>(dOs, QSTR, 16 * db + c16, s * M::KSTEP, g);
          qtf = load_col_acc<T>(Qs, QSTR, 16 * db + c16, s * M::KSTEP, g);
        }
#pragma unroll
        for (int jb = 0; jb < 2; ++jb) {
          dva[db][jb] = M::mma(dof, pf[jb], dva[db][jb]);
          dka[db][jb] = M::mma(qtf, df[jb], dka[db][jb]);
        }
      }
    }

    // ---- p2c gradients: dK += dSp^T Qr, dQr += dSp K ------------------------------------
    if (p.flags & 2) {
      int tmin, tmax;
      wave_rel_range(tbl, 0, BQ + BKW - 1, l, tmin, tmax);
      const int pmin = p2c_row(tmax, A), pmax = p2c_row(tmin, A);
      int wmin, wmax;
      wave_rel_range(tbl, (BKW - 1) - w * WK - 31, WK + BQ - 1, l, wmin, wmax);
      const int pwmin = p2c_row(wmax, A), pwmax = p2c_row(wmin, A);
      for (int pb = pmin; pb <= pmax; pb += WB) {
        const int nrow = min(WB, pmax - pb + 1);
        __syncthreads();
        for (int x = tid; x < nrow * (BKW / 4); x += 256) {
          reinterpret_cast<f32x4*>(band)[(x / (BKW / 4)) * (WB_STR / 4) + (x % (BKW / 4))] = zero4();
        }
        __syncthreads();
#pragma unroll
        for (int jb = 0; jb < 2; ++jb)
#pragma unroll
          for (int ib = 0; ib < 4; ++ib)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float v = ds[jb][ib][e];
              if (v != 0.f) {
                const int xi = (16 * ib + 4 * g + e) - (w * WK + 16 * jb + c16) + (BKW - 1);
                const int r = p2c_row(tbl[xi], A) - pb;
                if (r >= 0 && r < nrow) atomicAdd(&band[r * WB_STR + w * WK + 16 * jb + c16], v);
              }
            }
        __syncthreads();
        // dK^T[d, j] += sum_r QrT[d, r] band[r, j] over this wave's keys
        {
          const int lo = max(pwmin, pb) - pb, hi = min(pwmax, pb + nrow - 1) - pb;
          if (lo <= hi) {
            const int rs0 = ((pb + lo) / M::KSTEP) * M::KSTEP;
            for (int rs = rs0; rs <= pb + hi; rs += M::KSTEP) {
              frag bfr[2];
#pragma unroll
              for (int jb = 0; jb < 2; ++jb) bfr[jb] = band_col_frag<T>(band, w * WK + 16 * jb + c16, rs - pb, lo, hi, g);
#pragma unroll
              for (int db = 0; db < ND; ++db) {
                const frag af = M::load_contig(qrTh + (int64_t)(16 * db + c16) * bp.Rpad + rs, 0, g);
#pragma unroll
                for (int jb = 0; jb < 2; ++jb) dka[db][jb] = M::mma(af, bfr[jb], dka[db][jb]);
              }
            }
          }
        }
        // dQr[r, d] += sum_j band[r, j] K[j, d] for the blocks this wave owns
        {
          const int blo = pb >> 4, bhi = (pb + nrow - 1) >> 4;
          for (int rbg = blo + ((w - blo % NW) + NW) % NW; rbg <= bhi; rbg += NW) {
            f32x4 res[ND];
#pragma unroll
            for (int db = 0; db < ND; ++db) res[db] = zero4();
            const int row = 16 * rbg + c16 - pb;
#pragma unroll
            for (int s = 0; s < BKW / M::KSTEP; ++s) {
              const frag af = band_row_frag<T>(band, row, nrow, s * M::KSTEP, g);
#pragma unroll
              for (int db = 0; db < ND; ++db) {
                frag ktf;
                if constexpr (BF) {
                  ktf = M::load_contig(&Kt[(16 * db + c16) * KTSTR], s, g);
                } else {
#pragma unroll
                  for (int e = 0; e < 4; ++e) {
                    const int j = j0 + s * M::KSTEP + 4 * g + e;
                    ktf[e] = (j < Lk) ? kbase[(int64_t)j * p.ks[1] + 16 * db + c16] : 0.f;
                  }
                }
                res[db] = M::mma(af, ktf, res[db]);
              }
            }
            const int slot = rbg / NW;
            bool held = false;
#pragma unroll
            for (int k = 0; k < OWN_SLOTS; ++k) {
              if (slot == k) {
#pragma unroll
                for (int db = 0; db < ND; ++db) dqra[k][db] += res[db];
                held = true;
              }
            }
            if (held) {
              touched |= 1u << slot;
            } else {
#pragma unroll
              for (int db = 0; db < ND; ++db) res[db] *= p.scale;
              atomic_add_block<D>(bp.dqr + (int64_t)h * R * D, R, 16 * rbg, res, g, c16);
            }
          }
        }
      }
      __syncthreads();
    }
  }

  // ---- epilogue --------------------------------------------------------------------------
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
  if (p.flags & 2) {
#pragma unroll
    for (int k = 0; k < OWN_SLOTS; ++k) {
      if (touched & (1u << k)) {
#pragma unroll
        for (int db = 0; db < ND; ++db) dqra[k][db] *= p.scale;
        atomic_add_block<D>(bp.dqr + (int64_t)h * R * D, R, 16 * (NW * k + w), dqra[k], g, c16);
      }
    }
  }
}

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

// dst[h, d, r] = src[h, r, d] for r < R, 0 for R <= r < Rpad
template <typename T, int D>
__global__ __launch_bounds__(256) void dsa_transpose_table_kernel(const T* src, int64_t sh, int64_t sr, T* dst,
                                                                  int H, int R, int Rpad) {
  const int64_t n = (int64_t)H * D * Rpad;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= n) return;
  const int r = (int)(idx % Rpad);
  const int d = (int)((idx / Rpad) % D);
  const int h = (int)(idx / ((int64_t)Rpad * D));
  dst[idx] = (r < R) ? src[(int64_t)h * sh + (int64_t)r * sr + d] : (T)0.0f;
}

}  // namespace dsa
