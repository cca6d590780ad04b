// dsa_bwd_dkp.h — the p2c term of dK from the stored dS^T (gfx950):
//
//   dK[j] = s (dKc[j] + sum_i dS_ij Qr[p(i-j)])
//
// where dKc is the content part Q^T dS that dsa_bwd_dkdv_kernel leaves in
// the workspace (fp32, unscaled).  One workgroup = 4 waves = one (batch b,
// head h, 128-key tile); wave w owns keys [jw, jw + 32), jw = j0 + 32w, and
// streams 64-query tiles of dS^T and the tile's qrgt window through LDS
// (the next tile is fetched into registers while the current one is
// computed):
//   dK^T[d][j] += sum_x qrgt[d][t0 + x] F[x][j],   F[x][j] = dS^T[j][j + x - 31 + i0 - jw]
// with x = (i - i0) - (j - jw) + 31 the wave's offset index and qrgt the Qr
// rows gathered per offset and transposed.  Row j of dS^T is contiguous in
// i, so F's operand is eight consecutive elements of one LDS row; 32 zero
// columns on either side of the tile cover offsets outside it.
#pragma once

#include "dsa_bwd.h"

namespace dsa {

namespace dkpcfg {
constexpr int NW = 4, WK = 32, BKW = 128, BQ = 64;
constexpr int XW = 96;   // offset rows per wave (95 used)
constexpr int ZC = 32;   // zero columns on either side of the tile
}  // namespace dkpcfg

template <typename T, int D>
__global__ __launch_bounds__(256, 2) void dsa_bwd_dkp_kernel(BwdParams bp) {
  using namespace dkpcfg;
  using M = Mfma<T>;
  typedef typename M::frag frag;
  constexpr int VEC = 16 / sizeof(T);
  typedef T vecT __attribute__((ext_vector_type(VEC)));
  constexpr int ND = D / 16;
  constexpr int FE = M::FRAG_ELEMS;
  constexpr int TSTR = ZC + BQ + ZC + Pad<T>::v;
  constexpr int GW = BKW - WK + XW;            // qrgt columns of the workgroup's window (192)
  constexpr int GSTR = GW + Pad<T>::v;
  constexpr int TV = BKW * BQ / VEC, GV = D * GW / VEC;  // 16-byte chunks per tile
  constexpr int TCH = (TV + 255) / 256, GCH = (GV + 255) / 256;
  const FwdParams& p = bp.f;

  __shared__ __align__(16) T Ts[BKW * TSTR];
  __shared__ __align__(16) T QG[D * GSTR];

  const int tid = threadIdx.x;
  const int w = tid >> 6, g = (tid & 63) >> 4, c16 = tid & 15;
  const int kt = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int j0 = kt * BKW, jw = j0 + w * WK;
  const T* dsb = (const T*)bp.dst + ((int64_t)(b * p.H + h) * bp.f.LkP + j0) * bp.f.LqP;
  const T* qrg = (const T*)bp.qrgt + (int64_t)h * D * bp.TGP;

  // zero columns (never overwritten)
  for (int c = tid; c < BKW * 2 * ZC / VEC; c += 256) {
    const int r = c / (2 * ZC / VEC), k = c % (2 * ZC / VEC);
    const int col = (k < ZC / VEC) ? k * VEC : ZC + BQ + (k - ZC / VEC) * VEC;
    vecT z;
#pragma unroll
    for (int e = 0; e < VEC; ++e) z[e] = (T)0.0f;
    *reinterpret_cast<vecT*>(Ts + r * TSTR + col) = z;
  }

  f32x4 acc[ND][2];
#pragma unroll
  for (int db = 0; db < ND; ++db) acc[db][0] = acc[db][1] = zero4();

  const int nqt = bp.f.LqP / BQ;
  // The next query tile (dS^T columns and the qrgt window) is fetched into
  // registers while the current one is computed.
  vecT xr[TCH], gr[GCH];
  auto fetch = [&](int qi) {
#pragma unroll
    for (int k = 0; k < TCH; ++k) {
      const int c = tid + 256 * k;
      if (c < TV) {
        const int r = c / (BQ / VEC), c0 = (c % (BQ / VEC)) * VEC;
        xr[k] = *reinterpret_cast<const vecT*>(dsb + (int64_t)r * bp.f.LqP + qi * BQ + c0);
      }
    }
    const int tw = qi * BQ - j0 - (BKW - 1) + bp.OFF;  // window column 0 (a multiple of 32)
#pragma unroll
    for (int k = 0; k < GCH; ++k) {
      const int c = tid + 256 * k;
      if (c < GV) gr[k] = *reinterpret_cast<const vecT*>(qrg + (int64_t)(c / (GW / VEC)) * bp.TGP + tw + (c % (GW / VEC)) * VEC);
    }
  };
  fetch(0);
  for (int qi = 0; qi < nqt; ++qi) {
    __syncthreads();  // previous tile's readers are done
#pragma unroll
    for (int k = 0; k < TCH; ++k) {
      const int c = tid + 256 * k;
      if (c < TV) *reinterpret_cast<vecT*>(Ts + (c / (BQ / VEC)) * TSTR + ZC + (c % (BQ / VEC)) * VEC) = xr[k];
    }
#pragma unroll
    for (int k = 0; k < GCH; ++k) {
      const int c = tid + 256 * k;
      if (c < GV) *reinterpret_cast<vecT*>(QG + (c / (GW / VEC)) * GSTR + (c % (GW / VEC)) * VEC) = gr[k];
    }
    __syncthreads();
    if (qi + 1 < nqt) fetch(qi + 1);

    // qrgt column of x = 0 for this wave: i0 - jw - 31 + OFF, i.e. window column 96 - 32w
#pragma unroll
    for (int s = 0; s < XW / M::KSTEP; ++s) {
      frag bfr[2];
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) {
        // k = x = KSTEP*s + FE*g + e  ->  tile column i = x + j_local - 31
        const int jl = 16 * jb + c16;
        const T* row = Ts + (WK * w + jl) * TSTR + ZC + M::KSTEP * s + FE * g + jl - 31;
#pragma unroll
        for (int e = 0; e < FE; ++e) bfr[jb][e] = row[e];
      }
#pragma unroll
      for (int db = 0; db < ND; ++db) {
        const frag af = M::load_contig(QG + (16 * db + c16) * GSTR + BKW - WK - WK * w, s, g);
#pragma unroll
        for (int jb = 0; jb < 2; ++jb) acc[db][jb] = M::mma(af, bfr[jb], acc[db][jb]);
      }
    }
  }

  // dK = s (dKc + p2c term); lanes hold 4 consecutive head-dim columns of key j
  const float* dkc = bp.dkc + ((int64_t)(b * p.H + h) * bp.f.LkP) * D;
  T* dkbase = (T*)bp.dk + (int64_t)b * bp.dks[0] + (int64_t)h * bp.dks[2];
#pragma unroll
  for (int jb = 0; jb < 2; ++jb) {
    const int j = jw + 16 * jb + c16;
    if (j < p.Lk) {
#pragma unroll
      for (int db = 0; db < ND; ++db) {
        const f32x4 c = *reinterpret_cast<const f32x4*>(dkc + (int64_t)j * D + 16 * db + 4 * g);
        typedef T vec4 __attribute__((ext_vector_type(4)));
        vec4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (T)((c[e] + acc[db][jb][e]) * p.scale);
        *reinterpret_cast<vec4*>(dkbase + (int64_t)j * bp.dks[1] + 16 * db + 4 * g) = v;
      }
    }
  }
}

}  // namespace dsa
