// dsa_fwd.h — fused disentangled-attention forward kernel (gfx950).
//
// One workgroup = 4 waves = one (batch b, head h, 128-query tile).  Wave w
// owns queries [i0 + 32w, i0 + 32w + 32) and streams 64-key tiles:
//
//   S^T = K Q^T                      MFMA, K tile from LDS, Q^T in registers
//   + c2p band (per wave)            MFMA  Kr[c(x)] Q^T  -> LDS (fp16) -> gather
//   + p2c band (per workgroup)       MFMA  K Qr[p(x)]^T  -> LDS (fp16) -> gather
//   mask, online softmax (exp2)      fp32, per query column, with a lazily
//                                    raised reference max
//   O^T += V^T P^T                   MFMA, P fed from registers (ACC k-set),
//                                    V^T read transposed from LDS
// The next key tile is fetched into registers while the current one's
// softmax and PV product run (requested after its band rows).
//
// The score tile is kept transposed (keys down, queries across) so that the
// probabilities a lane holds are already the B operand of the PV product.
// The relative terms are computed per query/key offset x = i - j (see
// add_delta_bands_T): every score element reads its band value at a
// compile-time offset from a per-lane base.
#pragma once

#include "dsa_dropout.h"
#include "dsa_tiles.h"

namespace dsa {

// QC: the c2p term reads the query rows p.qc (which carry the p2p term)
// instead of q.  DROP: attention dropout with the keep bits p.drop
// (dsa_dropout.h): dropped probabilities leave the PV product, the row sums
// (and so the lse) keep them, and the output is scaled by p.drop_scale.
template <typename T, int D, int MASK, bool QC = false, bool DROP = false>
__global__ __launch_bounds__(256, 2) void dsa_fwd_kernel(FwdParams p) {
  using namespace dcfg;
  using M = Mfma<T>;
  typedef typename M::frag frag;
  typedef typename BandType<T>::type BT;
  constexpr int NS = D / M::KSTEP;        // k steps over the head dim
  constexpr int KSTR = D + Pad<T>::v;      // Ks / Vs row stride
  constexpr int ND = D / 16;               // 16-wide tiles over the head dim
  constexpr int PV_STEPS = BK / M::KSTEP;  // k steps over the key tile
  constexpr int VEC = 16 / sizeof(T);
  typedef T vecT __attribute__((ext_vector_type(VEC)));
  constexpr int KV = BK * D / VEC;         // 16-byte chunks of a K (or V) tile
  constexpr int KCH = (KV + 255) / 256;

  __shared__ __align__(16) T Ks[BK * KSTR];
  __shared__ __align__(16) T Vs[BK * KSTR];
  __shared__ int crow[XG], prow[XG];
  __shared__ __align__(16) BT cb_all[NW * CB_ELEMS];
  __shared__ __align__(16) BT pb[PB_ELEMS];
  constexpr bool SEGM = seg_mode(MASK);
  constexpr int MAXKT = 512;  // key tiles (Lk <= 32768)
  __shared__ int segred[SEGM ? 3 * NW : 1];
  __shared__ __align__(16) int ksg[SEGM ? BK : 1];  // key segments of the current tile
  // segment masks: per key tile, bit 0 = some pair of one segment, bit 1 =
  // no masking needed; the list of the active tiles in order
  __shared__ unsigned char kflag[SEGM ? MAXKT : 1];
  __shared__ short klist[SEGM ? MAXKT : 1];
  __shared__ int klen;

  const int tid = threadIdx.x;
  const int w = tid >> 6, g = (tid & 63) >> 4, c16 = tid & 15;
  const int NQT = (p.Lq + BQ - 1) / BQ;
  // (b, h, qt), qt fastest; with an order (masks), item order[r / H] and
  // head r % H, heaviest first
  int qt, h, b;
  if (p.order) {
    // one read of the item, shared through LDS, so that the whole workgroup
    // takes one decision; an item outside [0, B * NQT) (an order another
    // call overwrote meanwhile) ends the workgroup before it indexes
    // anything
    __shared__ int item;
    if (tid == 0) item = p.order[blockIdx.x / p.H];
    __syncthreads();
    const int it = item;
    if (it < 0 || it >= p.B * NQT) return;
    h = blockIdx.x % p.H, qt = it % NQT, b = it / NQT;
  } else {
    const int m = xcd_remap(blockIdx.x, gridDim.x);
    qt = m % NQT, h = (m / NQT) % p.H, b = m / (NQT * p.H);
  }
  const int Lq = p.Lq, Lk = p.Lk, A = p.A;
  const int i0 = qt * BQ;
  const int iw = i0 + w * WQ;
  BT* cb = cb_all + w * CB_ELEMS;

  const T* qbase = (const T*)p.q + (int64_t)b * p.qs[0] + (int64_t)h * p.qs[2];
  const T* kbase = (const T*)p.k + (int64_t)b * p.ks[0] + (int64_t)h * p.ks[2];
  const T* vbase = (const T*)p.v + (int64_t)b * p.vs[0] + (int64_t)h * p.vs[2];
  const T* krh = (p.flags & 1) ? (const T*)p.kr + (int64_t)h * p.krs[0] : nullptr;
  const T* qrh = (p.flags & 2) ? (const T*)p.qr + (int64_t)h * p.qrs[0] : nullptr;
  const uint8_t* pkb = (MASK == MASK_PAIR) ? p.pk + (int64_t)b * p.pkb + (int64_t)h * p.pkh : nullptr;
  const SegView<MASK> sv(p, b);

  // Per-lane query columns (two 16-wide tiles per wave) and their segments.
  int irow[2], sq[2] = {0, 0};
  bool ilive[2];
#pragma unroll
  for (int ib = 0; ib < 2; ++ib) {
    irow[ib] = iw + 16 * ib + c16;
    bool valid = irow[ib] < Lq;
    bool live = valid;
    if (SEGM && valid) {
      sq[ib] = sv(irow[ib]);
      live = sq[ib] != 0;
    }
    if (MASK == MASK_PAIR && valid) live = pkb[(int64_t)irow[ib] * p.pkq + irow[ib]] != 0;
    ilive[ib] = live;
  }

  // Q^T fragments stay in registers for the whole key loop.
  frag qf[2][NS];
#pragma unroll
  for (int ib = 0; ib < 2; ++ib)
#pragma unroll
    for (int s = 0; s < NS; ++s)
      qf[ib][s] = (irow[ib] < Lq) ? M::load_contig(qbase + (int64_t)irow[ib] * p.qs[1], s, g) : M::zero();
  // the c2p term's query rows (QC: qc, else the same Q^T fragments)
  frag qcf[2][NS];
  if constexpr (QC) {
    const T* qcbase = (const T*)p.qc + (int64_t)b * p.qcs[0] + (int64_t)h * p.qcs[2];
#pragma unroll
    for (int ib = 0; ib < 2; ++ib)
#pragma unroll
      for (int s = 0; s < NS; ++s)
        qcf[ib][s] = (irow[ib] < Lq) ? M::load_contig(qcbase + (int64_t)irow[ib] * p.qcs[1], s, g) : M::zero();
  }

  float mref[2] = {-INFINITY, -INFINITY};  // reference max of the unscaled scores
  float lrow[2] = {0.f, 0.f};
  f32x4 o[ND][2];
#pragma unroll
  for (int db = 0; db < ND; ++db) o[db][0] = o[db][1] = zero4();

  const float sl2 = p.scale * kLog2e;
  const float thr = 8.f / sl2;  // reference-max slack (unscaled): p <= 2^8
  const int nkt = (Lk + BK - 1) / BK;
  // this lane's first element of the saved relative term in each key tile
  BT* biasl = (p.bias && p.flags) ? (BT*)p.bias + bias_tile_offset(b, h, p.H, qt, 0, p.LqP, p.LkP) + w * 2048 +
                                        c16 * 16 + g * 4
                                  : nullptr;

  // Is any query row of this workgroup live?  If not, nothing to compute.
  // Segment masks: the range of the workgroup's query segments decides
  // which key tiles can hold kept pairs.
  SegRange qsr{0, -1, false};
  bool any_live;
  if constexpr (SEGM) {
    const int i = i0 + tid;
    qsr = wg_seg_range((tid < BQ && i < Lq) ? sv(i) : 0, tid < BQ, segred);
    any_live = qsr.any();
  } else {
    int wg_live = 0;
    if (tid < BQ) {
      int i = i0 + tid;
      if (i < Lq) wg_live = (MASK == MASK_NONE) ? 1 : pkb[(int64_t)i * p.pkq + i] != 0;
    }
    any_live = __syncthreads_or(wg_live);
  }

  // Segment masks: the key tiles with a kept pair (a key whose segment is
  // one of the workgroup's query segments), found once from the key
  // segments (wave w tests tiles w, w + 4, ..., eight at a time), and
  // listed in order; the loop visits only those.
  int nlist = nkt;
  if constexpr (SEGM) {
    static_assert(BK == 64, "one key of a tile per lane");
    if (any_live) {
      const bool one = qsr.all && qsr.lo == qsr.hi;  // every query in one segment
      const int lane = tid & 63;
      for (int u0 = 0; u0 < nkt; u0 += 4 * 8) {
        int s8[8];
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          const int j = (u0 + 4 * v + w) * BK + lane;
          s8[v] = j < Lk ? sv(j) : 0;
        }
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          const int kt = u0 + 4 * v + w;
          const bool act = __ballot(qsr.meets(s8[v])) != 0;
          const bool full = one && __ballot(s8[v] != qsr.lo) == 0;
          if (lane == 0 && kt < nkt) kflag[kt] = (act ? 1 : 0) | (act && full ? 2 : 0);
        }
      }
    }
    __syncthreads();
    if (w == 0) {
      const int lane = tid & 63;
      int n = 0;
      for (int c0 = 0; any_live && c0 < nkt; c0 += 64) {
        const int c = c0 + lane;
        n = wave_append(c < nkt && (kflag[c] & 1), (short)c, klist, n);
      }
      if (lane == 0) klen = n;
    }
    __syncthreads();
    nlist = __builtin_amdgcn_readfirstlane(klen);
  }

  // The next key tile (K and V rows) is fetched into registers while the
  // current one's softmax and PV product run.
  vecT kr[KCH], vr[KCH];
  int relv = 0;  // this thread's relative position of the fetched tile (tid < XG)
  int ksn = 0;   // segment masks: this thread's key segment of the fetched tile (tid < BK)
  int kfetched = -1;
  // dropout: this lane's keep word of the fetched tile (bit 16 ib + 4 jb + e)
  uint32_t dwn = 0;
  const uint32_t* dropw = nullptr;
  if constexpr (DROP) {
    static_assert(BK == 64 && WQ == 32, "one keep word per lane, 32-query block and 64-key tile");
    dropw = p.drop + drop_word0(b, h, p.H, p.LqP / 32, p.LkP / 64, iw / 32, 0) + (tid & 63);
  }
  auto fetch = [&](int kt) {
    const int j0 = kt * BK;
    if constexpr (DROP) dwn = dropw[(int64_t)kt * 64];
    if (p.flags && tid < XG) relv = rel_of_tile(p.rel, i0, j0, Lq, Lk, tid);
    if (SEGM && tid < BK) ksn = j0 + tid < Lk ? sv(j0 + tid) : 0;
#pragma unroll
    for (int k = 0; k < KCH; ++k) {
      const int c = tid + 256 * k;
      const int j = j0 + c / (D / VEC), c0 = (c % (D / VEC)) * VEC;
#pragma unroll
      for (int e = 0; e < VEC; ++e) kr[k][e] = vr[k][e] = (T)0.0f;
      if (c < KV && j < Lk) {
        kr[k] = *reinterpret_cast<const vecT*>(kbase + (int64_t)j * p.ks[1] + c0);
        vr[k] = *reinterpret_cast<const vecT*>(vbase + (int64_t)j * p.vs[1] + c0);
      }
    }
    kfetched = kt;
  };
  if (any_live && nlist > 0) fetch(SEGM ? __builtin_amdgcn_readfirstlane(klist[0]) : 0);
  // The Q fragments and the first tile have landed before the loop (its
  // first iteration waits for the tile anyway).  Without this wait the
  // loads issued before the loop stay pending in the compiler's view of the
  // loop, and the first score product of every tile waited for all
  // outstanding loads: the next tile's prefetch included.
  vm_wait<0>();

  for (int n = 0; any_live && n < nlist; ++n) {
    const int kt = SEGM ? __builtin_amdgcn_readfirstlane(klist[n]) : n;
    const int j0 = kt * BK;
    // Skip key tiles that every query row of the workgroup masks out: their
    // probabilities are exactly zero (segment masks: the list holds the
    // others).  With segments, a tile whose keys all share the workgroup's
    // single query segment needs no masking at all.
    bool full = false;
    if constexpr (SEGM) {
      full = (kflag[kt] & 2) != 0;
    } else if (MASK == MASK_PAIR) {
      // 16-byte reads of the mask rows (rows 16-byte aligned, host-checked;
      // a 16-key chunk that starts below Lk lies in the row's allocation)
      uint32_t keep = 0;
      const int r = tid >> 1, half = tid & 1;
      const int i = i0 + r;
      if (i < Lq) {
        const uint8_t* row = pkb + (int64_t)i * p.pkq;
#pragma unroll
        for (int c = 0; c < BK / 32; ++c) {
          const int jc = j0 + half * (BK / 2) + 16 * c;
          if (jc < Lk) {
            const uint4 v = *reinterpret_cast<const uint4*>(row + jc);
            keep |= v.x | v.y | v.z | v.w;
          }
        }
      }
      if (!__syncthreads_or(keep != 0)) continue;
    }
    __syncthreads();  // previous tile's LDS reads are done
    // Everything this wave requested in the previous tile has landed or been
    // written by now (the prefetch and the saved-term stores were issued
    // before its softmax and PV product).  Waiting here, unconditionally,
    // tells the compiler so: with stores and loads both outstanding it
    // cannot order them, and would otherwise wait for everything at the
    // first reuse of a register that an earlier load wrote.
    vm_wait<0>();
    if (kt != kfetched) fetch(kt);  // a tile after skipped ones was not prefetched
    uint32_t dw = 0;
    if constexpr (DROP) dw = dwn;  // the next fetch overwrites dwn
#pragma unroll
    for (int k = 0; k < KCH; ++k) {
      const int c = tid + 256 * k;
      if (c < KV) {
        const int r = c / (D / VEC), c0 = (c % (D / VEC)) * VEC;
        *reinterpret_cast<vecT*>(Ks + r * KSTR + c0) = kr[k];
        *reinterpret_cast<vecT*>(Vs + r * KSTR + c0) = vr[k];
      }
    }
    if (SEGM && tid < BK) ksg[tid] = ksn;
    if (p.flags) store_row_tables(crow, prow, relv, A, (int)p.krs[1], (int)p.qrs[1], tid);
    __syncthreads();

    // ---- y = K Q^T + c2p + p2c (unscaled) -------------------------------------
    frag kf[4][NS];
#pragma unroll
    for (int jb = 0; jb < 4; ++jb)
#pragma unroll
      for (int s = 0; s < NS; ++s) kf[jb][s] = M::load_contig(&Ks[(16 * jb + c16) * KSTR], s, g);
    // The score and band products, and the PV product below, run at a
    // raised wave priority, so that the SIMD's other wave fills in with its
    // softmax (VALU) work (forward 144.8 -> 143.7 us in one process).
    f32x4 st[2][4];
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int jb = 0; jb < 4; ++jb)
#pragma unroll
      for (int ib = 0; ib < 2; ++ib) {
        f32x4 acc = zero4();
#pragma unroll
        for (int s = 0; s < NS; ++s) acc = M::mma(kf[jb][s], qf[ib][s], acc);
        st[ib][jb] = acc;
      }
    // The next tile is requested only after this tile's band rows have been
    // waited for (a wave's vector-memory requests complete in issue order,
    // so a request issued before them would be waited for with them) and
    // before the saved-term stores (with stores outstanding the compiler
    // cannot order the counts and waits for everything).  It has the gather,
    // the softmax and the PV product to land.
    if (p.flags)
      band_products_T<T, D, MASK == MASK_PAIR ? 3 : 6>(kf, pick<QC>(qcf, qf), cb, pb, crow, prow, w, g, c16, krh, qrh,
                                                       p.krk, p.qrk, p.flags);
    if (n + 1 < nlist) fetch(SEGM ? __builtin_amdgcn_readfirstlane(klist[n + 1]) : n + 1);
    if (p.flags) band_gather_T<T, D>(st, cb, pb, w, g, c16, p.flags, biasl ? biasl + (int64_t)kt * 8192 : nullptr);
    __builtin_amdgcn_s_setprio(0);

    // ---- mask: only where a key or query of the tile can be masked out ------
    if (MASK == MASK_PAIR || (SEGM && !full) || j0 + BK > Lk) {
#pragma unroll
      for (int ib = 0; ib < 2; ++ib) {
        const int i = irow[ib];
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
          int4 ks4 = {0, 0, 0, 0};
          if constexpr (SEGM) ks4 = *reinterpret_cast<const int4*>(&ksg[16 * jb + 4 * g]);
          uint32_t pk4 = 0;
          if (MASK == MASK_PAIR && ilive[ib]) {
            const int j = j0 + 16 * jb + 4 * g;
            if (j < Lk) {  // one 4-byte read: keys j .. j + 3 (j < Lk covers them, as above)
              const uint32_t v = *reinterpret_cast<const uint32_t*>(pkb + (int64_t)i * p.pkq + j);
#pragma unroll
              for (int e = 0; e < 4; ++e) pk4 |= ((v >> (8 * e)) & 0xffu) ? (1u << e) : 0u;
            }
          }
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int j = j0 + 16 * jb + 4 * g + e;
            bool keep = ilive[ib] && j < Lk;
            if constexpr (SEGM) keep = keep && sq[ib] == (e == 0 ? ks4.x : e == 1 ? ks4.y : e == 2 ? ks4.z : ks4.w);
            if (MASK == MASK_PAIR) keep = keep && ((pk4 >> e) & 1u);
            if (!keep) st[ib][jb][e] = -INFINITY;
          }
        }
      }
    }

    // ---- online softmax -------------------------------------------------------
    // Scores stay unscaled; p = exp2((y - m) * scale*log2e) against a
    // reference max m per query that is raised (and O, l rescaled) only when
    // a score exceeds it by more than thr, so p <= 2^8.  Queries whose keys
    // are all masked so far keep m = -inf and p = 0.
    float lm[2];
    bool raise = false;
#pragma unroll
    for (int ib = 0; ib < 2; ++ib) {
      float mt = -INFINITY;
#pragma unroll
      for (int jb = 0; jb < 4; ++jb)
#pragma unroll
        for (int e = 0; e < 4; ++e) mt = fmaxf(mt, st[ib][jb][e]);
      lm[ib] = mt;
      raise = raise || mt > mref[ib] + thr;
    }
    if (__any(raise)) {
#pragma unroll
      for (int ib = 0; ib < 2; ++ib) {
        const float mnew = fmaxf(mref[ib], col_max(lm[ib]));
        const float alpha = (mref[ib] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f((mref[ib] - mnew) * sl2);
        lrow[ib] *= alpha;
#pragma unroll
        for (int db = 0; db < ND; ++db) o[db][ib] *= alpha;
        mref[ib] = mnew;
      }
    }
#pragma unroll
    for (int ib = 0; ib < 2; ++ib) {
      const float mb = (mref[ib] == -INFINITY) ? 0.f : mref[ib] * sl2;
      float ls = 0.f;
#pragma unroll
      for (int jb = 0; jb < 4; ++jb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float pe = __builtin_amdgcn_exp2f(__builtin_fmaf(st[ib][jb][e], sl2, -mb));
          st[ib][jb][e] = pe;
          ls += pe;
        }
      lrow[ib] += ls;
    }
    if constexpr (DROP) {
      // dropped probabilities leave the PV product (after the row sums)
#pragma unroll
      for (int ib = 0; ib < 2; ++ib)
#pragma unroll
        for (int jb = 0; jb < 4; ++jb)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (!((dw >> (16 * ib + 4 * jb + e)) & 1u)) st[ib][jb][e] = 0.f;
    }

    // ---- O^T += V^T P^T -------------------------------------------------------
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int s = 0; s < PV_STEPS; ++s) {
      frag pf[2];
#pragma unroll
      for (int ib = 0; ib < 2; ++ib) pf[ib] = M::from_acc(st[ib], s);
#pragma unroll
      for (int db = 0; db < ND; ++db) {
        const frag vf = tr_acc<T>(Vs, KSTR, s * M::KSTEP, 16 * db, g, c16);
#pragma unroll
        for (int ib = 0; ib < 2; ++ib) o[db][ib] = M::mma(vf, pf[ib], o[db][ib]);
      }
    }
    __builtin_amdgcn_s_setprio(0);
  }

  // ---- epilogue -----------------------------------------------------------
  T* obase = (T*)p.out + (int64_t)b * p.os[0] + (int64_t)h * p.os[2];
#pragma unroll
  for (int ib = 0; ib < 2; ++ib) {
    const int i = irow[ib];
    const float lsum = col_sum(lrow[ib]);
    const bool ok = ilive[ib] && lsum > 0.f;
    const float inv = ok ? (DROP ? p.drop_scale : 1.f) / lsum : 0.f;
    if (i < Lq) {
      T* orow = obase + (int64_t)i * p.os[1];
      // bf16 with p.olo: also the rounding residual of each element, for
      // the backward's row sums dO . O (p.olo has out's strides: the same
      // byte offset from its base)
      T* lrow = (sizeof(T) == 2 && p.olo) ? (T*)((uintptr_t)orow + ((uintptr_t)p.olo - (uintptr_t)p.out)) : nullptr;
#pragma unroll
      for (int db = 0; db < ND; ++db) {
        typedef T vec4 __attribute__((ext_vector_type(4)));
        vec4 v, r;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float f = o[db][ib][e] * inv;
          v[e] = (T)f;
          r[e] = (T)(f - (float)v[e]);
        }
        *reinterpret_cast<vec4*>(orow + 16 * db + 4 * g) = v;
        if (lrow) *reinterpret_cast<vec4*>(lrow + 16 * db + 4 * g) = r;
      }
      if (g == 0) p.lse[((int64_t)b * p.H + h) * Lq + i] = ok ? (mref[ib] * p.scale + logf(lsum)) : INFINITY;
    }
  }
}

}  // namespace dsa
