// dsa_bias.h — the relative score term alone (gfx950): the reference's bias
// API DisentangledSelfAttention.disentangled_attention_bias
// (deberta_v2_native.py:530-562 over :349-432 / :434-528), which returns
//   bias[b, h, i, j] = (c2p(i, j) + p2c(i, j) [+ p2p(i, j)]) / sqrt(D * sf)
// as a (B, H, Lq, Lk) tensor, unmasked.
//
// One workgroup = 4 waves = one (b, h, 128-query tile, 64-key tile), the
// forward's tile: the band products of add_delta_bands_T (the forward's
// own code for the relative terms) on a zero score tile, scaled and written
// row-major.  The p2p term rides on the c2p term's query rows (qc), as in
// the forward.
#pragma once

#include "dsa_tiles.h"

namespace dsa {

struct BiasParams {
  FwdParams f;
  void* out;        // [B, H, Lq, Lk], dtype of q, unit stride over j
  int64_t obs[3];   // element strides of b, h, i
};

template <typename T, int D, bool QC>
__global__ __launch_bounds__(256, 2) void dsa_bias_kernel(BiasParams bp) {
  using namespace dcfg;
  using M = Mfma<T>;
  typedef typename M::frag frag;
  typedef typename BandType<T>::type BT;
  constexpr int NS = D / M::KSTEP;
  __shared__ int crow[XG], prow[XG];
  __shared__ __align__(16) BT cb_all[NW * CB_ELEMS];
  __shared__ __align__(16) BT pb[PB_ELEMS];

  const FwdParams& p = bp.f;
  const int tid = threadIdx.x;
  const int w = tid >> 6, g = (tid & 63) >> 4, c16 = tid & 15;
  const int Lq = p.Lq, Lk = p.Lk;
  const int NQT = (Lq + BQ - 1) / BQ, NKT = (Lk + BK - 1) / BK;
  int m = blockIdx.x;
  const int kt = m % NKT;
  m /= NKT;
  const int qt = m % NQT;
  m /= NQT;
  const int h = m % p.H, b = m / p.H;
  const int i0 = qt * BQ, j0 = kt * BK, iw = i0 + w * WQ;

  // the c2p term's query rows (qc carries p2p) and the tile's keys, as
  // operand fragments read straight from memory (zero past the ends)
  const T* qsrc = (const T*)(QC ? p.qc : p.q);
  const int64_t* qst = QC ? p.qcs : p.qs;
  const T* qbase = qsrc + (int64_t)b * qst[0] + (int64_t)h * qst[2];
  const T* kbase = (const T*)p.k + (int64_t)b * p.ks[0] + (int64_t)h * p.ks[2];
  frag qf[2][NS], kf[4][NS];
#pragma unroll
  for (int ib = 0; ib < 2; ++ib) {
    const int i = iw + 16 * ib + c16;
#pragma unroll
    for (int s = 0; s < NS; ++s) qf[ib][s] = i < Lq ? M::load_contig(qbase + (int64_t)i * qst[1], s, g) : M::zero();
  }
#pragma unroll
  for (int jb = 0; jb < 4; ++jb) {
    const int j = j0 + 16 * jb + c16;
#pragma unroll
    for (int s = 0; s < NS; ++s) kf[jb][s] = j < Lk ? M::load_contig(kbase + (int64_t)j * p.ks[1], s, g) : M::zero();
  }
  if (p.flags && tid < XG)
    store_row_tables(crow, prow, rel_of_tile(p.rel, i0, j0, Lq, Lk, tid), p.A, (int)p.krs[1], (int)p.qrs[1], tid);
  __syncthreads();

  f32x4 y[2][4];
#pragma unroll
  for (int ib = 0; ib < 2; ++ib)
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) y[ib][jb] = zero4();
  if (p.flags) {
    const T* krh = (p.flags & 1) ? (const T*)p.kr + (int64_t)h * p.krs[0] : nullptr;
    const T* qrh = (p.flags & 2) ? (const T*)p.qr + (int64_t)h * p.qrs[0] : nullptr;
    add_delta_bands_T<T, D, 6>(y, kf, qf, cb_all + w * CB_ELEMS, pb, crow, prow, w, g, c16, krh, qrh, p.krk, p.qrk,
                               p.flags);
  }

  // lane: query iw + 16 ib + c16, keys j0 + 16 jb + 4 g + [0, 4)
  typedef T vec4 __attribute__((ext_vector_type(4)));
  T* obase = (T*)bp.out + (int64_t)b * bp.obs[0] + (int64_t)h * bp.obs[1];
#pragma unroll
  for (int ib = 0; ib < 2; ++ib) {
    const int i = iw + 16 * ib + c16;
    if (i >= Lq) continue;
    T* orow = obase + (int64_t)i * bp.obs[2];
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      const int j = j0 + 16 * jb + 4 * g;
      vec4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = (T)(y[ib][jb][e] * p.scale);
      T* dst = orow + j;
      if (j + 3 < Lk && ((uintptr_t)dst % sizeof(vec4)) == 0) {
        *reinterpret_cast<vec4*>(dst) = v;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (j + e < Lk) dst[e] = v[e];
      }
    }
  }
}

}  // namespace dsa
