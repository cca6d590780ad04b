// dsa_bwd_dkdv.h — dK, dV and dS of the fused disentangled attention
// (gfx950).
//
// One workgroup = 4 waves = one (batch b, head h, 128-key tile); wave w owns
// keys [j0 + 32w, j0 + 32w + 32) and streams 32-query tiles.  The tiles (Q,
// dO, the saved relative term, lse and Delta, and a 32-offset block of
// qrgt) are double-buffered in LDS and filled by direct global-to-LDS copies
// issued one tile ahead; K and V of the wave's keys stay in registers.  Per
// tile:
//   scores        y = Q K^T + bias (unscaled), queries down / keys across,
//                 where bias = c2p + p2c is the relative term the forward
//                 saved (read transposed from the LDS tile)
//   P, dP, dS     P = exp2(y * scale*log2e - lse*log2e), dP = dO V^T,
//                 dS = P (dP - Delta)
//   dS            staged transposed in the wave's LDS tile (rows j), then
//                 stored to the workspace in rows i (4 consecutive keys per
//                 lane, read back transposed): the dq and table kernels
//                 read it
//   dV^T         += dO^T P,  dK^T += Q^T dS        (dO^T, Q^T read transposed)
//   p2c          dK^T[d][j] += sum_x qrgt[d][t0 + x] F[x][j], F[x][j] =
//                dS(i0 + x + (j - jw) - 31, j): x = (i - i0) - (j - jw) + 31 is
//                the wave's offset index and qrgt holds the Qr rows gathered
//                per offset and transposed.  The wave's dS^T tile in LDS
//                (rows j, 32 zero columns before each row) makes F's
//                operand eight consecutive elements of one row; the
//                qrgt window (160 offsets of the workgroup) is a ring of
//                32-offset blocks, one new block per tile.
// Every query tile of the padded extent is visited, so dS is fully written
// (zeros for masked pairs, dead rows and padding).
#pragma once

#include "dsa_bwd.h"
#include "dsa_dropout.h"

namespace dsa {

namespace kvcfg {
constexpr int NW = 4, WK = 32, BKW = 128, BQ = 32;
}  // namespace kvcfg

// DROP: attention dropout with the forward's keep bits p.drop
// (dsa_dropout.h): dV sums the kept probabilities, scaled by p.drop_scale,
// and dP keeps the kept pairs' dO . v, scaled the same way.
template <typename T, int D, int MASK, bool DROP = false>
__global__ __launch_bounds__(256, 2) void dsa_bwd_dkdv_kernel(BwdParams bp) {
  using namespace kvcfg;
  using M = Mfma<T>;
  typedef typename M::frag frag;
  typedef typename BandType<T>::type BT;
  using SQ = Swz<T, D>;
  constexpr int NS = D / M::KSTEP;
  constexpr int ND = D / 16;
  constexpr int VEC = 16 / (int)sizeof(T);
  constexpr int QCH = BQ * D * (int)sizeof(T) / 16;   // 16-byte chunks of a Q (or dO) tile
  constexpr int QCW = QCH / NW;                         // ... per wave
  constexpr int BE = 2 * 2048;                          // saved-bias elements of a tile
  constexpr int BCW = BE * (int)sizeof(BT) / 16 / NW;   // bias chunks per wave
  constexpr int FE = M::FRAG_ELEMS;
  // dS^T tile of a wave: rows j (32 + 1), ZL zero columns, 32 data columns,
  // the rest of the stride zero; a row's right-hand zeros continue into the
  // next row's leading ones.
  constexpr int ZL = 32;
  constexpr int SROW = sizeof(T) == 2 ? 72 : 76;         // few bank conflicts for 16-byte row reads
  constexpr int SW = (WK + 1) * SROW;
  // qrgt ring: NRB blocks of 32 offsets, each stored [chunk c][d][VEC] so that
  // a fragment read (one chunk of 16 consecutive d rows) is contiguous.
  constexpr int NRB = 6, RBE = 32 * D;
  constexpr int RCPB = RBE / VEC;                        // 16-byte chunks per block
  const FwdParams& p = bp.f;

  // Double-buffered tiles, filled by LDS copies issued one tile ahead.  The
  // two buffers are distinct arrays and the loop is unrolled by two, so the
  // compiler sees that a tile's reads do not touch the buffer the next
  // tile's copies are landing in (it would otherwise wait for those copies
  // before every read).
  __shared__ __align__(16) T Qs0[BQ * D], Qs1[BQ * D];
  __shared__ __align__(16) T dOs0[BQ * D], dOs1[BQ * D];
  __shared__ __align__(16) BT Bs0[BE], Bs1[BE];
  __shared__ __align__(16) float Rs0[2 * BQ], Rs1[2 * BQ];  // per query: lse*log2e (inf: no probabilities), Delta
  __shared__ __align__(16) T Ring[NRB * RBE];     // qrgt window (p2c)
  __shared__ __align__(16) T Stg[NW * SW];        // each wave's dS^T tile
  // dropout: each wave's keep words of the tile (one per lane), double-buffered
  __shared__ __align__(16) uint32_t Dk0[DROP ? NW * 64 : 1], Dk1[DROP ? NW * 64 : 1];
  constexpr bool SEGM = seg_mode(MASK);
  constexpr int MAXQT = 1024;  // query tiles (Lq <= 32768)
  // segment masks: the active query tiles in order (tile | 0x4000 if it
  // needs no masking); query segments of MASK_SEG tiles
  __shared__ short qlist[SEGM ? MAXQT : 1];
  __shared__ int qlen;
  __shared__ __align__(16) int qsg[MASK == MASK_SEG ? 2 : 1][MASK == MASK_SEG ? BQ : 1];
  // dense pair masks: the current tile's mask, one bit per (query, key),
  // 16 keys a word (read once per tile with 16-byte loads)
  __shared__ uint16_t pmask[MASK == MASK_PAIR ? BQ : 1][MASK == MASK_PAIR ? BKW / 16 : 1];

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = tid >> 6, g = (tid & 63) >> 4, c16 = tid & 15;
  const int Lq = p.Lq, Lk = p.Lk;
  const int NKT = p.LkP / BKW;
  // (b, h, kt), kt fastest; with an order (masks), item order[r / H] and
  // head r % H, heaviest first
  int kt, h, b;
  if (bp.korder) {
    const int it = bp.korder[blockIdx.x / p.H];
    h = blockIdx.x % p.H, kt = it % NKT, b = it / NKT;
  } else {
    const int m = xcd_remap(blockIdx.x, gridDim.x);
    kt = m % NKT, h = (m / NKT) % p.H, b = m / (NKT * p.H);
  }
  const bool p2c = (p.flags & 2) != 0;
  const float sl2 = p.scale * kLog2e;
  const int nqt = p.LqP / BQ;

  const int j0 = kt * BKW;
  const int jw = j0 + w * WK;
  const T* qbase = (const T*)p.q + (int64_t)b * p.qs[0] + (int64_t)h * p.qs[2];
  const T* kbase = (const T*)p.k + (int64_t)b * p.ks[0] + (int64_t)h * p.ks[2];
  const T* vbase = (const T*)p.v + (int64_t)b * p.vs[0] + (int64_t)h * p.vs[2];
  const T* dobase = (const T*)bp.dout + (int64_t)b * bp.dos[0] + (int64_t)h * bp.dos[2];
  const BT* biasb = (const BT*)p.bias;
  const float* rib = bp.rowinfo + (int64_t)(b * p.H + h) * p.LqP * 2;
  const uint8_t* pkb = (MASK == MASK_PAIR) ? p.pk + (int64_t)b * p.pkb + (int64_t)h * p.pkh : nullptr;
  const SegView<MASK> sv(p, b);
  T* dsw = (T*)bp.ds + (int64_t)(b * p.H + h) * p.LqP * p.LkP + jw;  // dS column jw, row 0
  const T* qrg = p2c ? (const T*)bp.qrgt + (int64_t)h * D * bp.TGP : nullptr;
  // qrgt column of the workgroup window's first offset at query tile 0
  // (a multiple of 32: t = d + OFF with d = -j0 - 127)
  const int tw0 = -j0 - (BKW - 1) + bp.OFF;
  T* stg = Stg + w * SW;

  int jcol[2], jseg[2] = {0, 0};
  bool jkeep[2];
#pragma unroll
  for (int jb = 0; jb < 2; ++jb) {
    const int j = jw + 16 * jb + c16;
    jcol[jb] = j;
    if (SEGM && j < Lk) jseg[jb] = sv(j);
    jkeep[jb] = j < Lk && (!SEGM || jseg[jb] != 0);
  }
  // Segment masks: the query tiles that meet this key tile (ChunkRange),
  // listed by wave 0 (one chunk per lane); the others are neither computed
  // nor written.
  bool any_key;
  int nlist = nqt;
  if constexpr (SEGM) {
    const ChunkRange kr = key_tile_range(bp.cinfo + (int64_t)b * nqt, kt, nqt);
    if (w == 0) {
      int n = 0;
      for (int c0 = 0; c0 < nqt; c0 += 64) {
        const int c = c0 + lane;
        bool act = false, full = false;
        if (c < nqt) {
          const ChunkRange x = chunk_range(bp.cinfo + (int64_t)b * nqt, c);
          act = x.meets(kr);
          full = act && x.all && kr.all && x.lo == x.hi && kr.lo == kr.hi && x.lo == kr.lo;
        }
        n = wave_append(act, (short)(c | (full ? 0x4000 : 0)), qlist, n);
      }
      if (lane == 0) qlen = n;
    }
    __syncthreads();
    nlist = __builtin_amdgcn_readfirstlane(qlen);
    any_key = nlist > 0;
  } else {
    any_key = __syncthreads_or(tid < BKW && j0 + tid < Lk);
  }

  f32x4 dka[ND][2], dva[ND][2];
#pragma unroll
  for (int db = 0; db < ND; ++db) dka[db][0] = dka[db][1] = dva[db][0] = dva[db][1] = zero4();

  // Issues the LDS copies of qrgt block rb (columns [32 rb, 32 rb + 32)) into
  // ring slot rb % NRB: chunk c of row d at ((c * D) + d) * VEC.
  typedef T vecT __attribute__((ext_vector_type(VEC)));
  auto issue_ring = [&](int rb) {
    T* slot = Ring + (rb % NRB) * RBE;
#pragma unroll
    for (int k = 0; k < (RCPB + 255) / 256; ++k) {
      const int pc = 256 * k + w * 64 + lane;
      if (256 * k + w * 64 < RCPB) {
        const int c = pc / D, d = pc % D;
        lds_dma16(qrg + (int64_t)d * bp.TGP + 32 * rb + c * VEC, (char*)(slot + (256 * k + w * 64) * VEC));
      }
    }
  };

  // Dropout: the forward's 64 keep words of the 32-query block qi and the
  // 64-key tile of the wave's keys (dsa_dropout.h), copied to LDS with the
  // tile (16 lanes x 16 bytes).  The pair (query i0 + 16 ib + 4 g + e, key
  // jw + 16 jb + c16) is bit 16 ib + 4 (2 (w % 2) + jb) + c16 % 4 of the word
  // of forward lane 16 (c16 / 4) + 4 g + e: a lane's four words are 16
  // contiguous bytes.
  const uint32_t* dropw = nullptr;
  const int NKT64 = p.LkP / 64;
  if constexpr (DROP) dropw = p.drop + drop_word0(b, h, p.H, p.LqP / 32, NKT64, 0, jw / 64);
  // Issues the LDS copies of query tile qi into the given buffers (lane
  // order = physical chunk order; Q and dO rows are clamped to Lq - 1, where
  // probabilities are zero anyway), and, with ring set, its qrgt block
  // (whose ring slot was last read two tiles earlier); with dropout, the
  // wave's keep words.
  int qseg_next = 0;  // MASK_SEG: query segment of lane (w = 1, lane < 32) in the next tile
  auto issue = [&](int qi, bool ring, T* Qd, T* dOd, BT* Bd, float* Rd, uint32_t* Dd) {
    const int i0 = qi * BQ;
    if (MASK == MASK_SEG && w == 1 && lane < BQ) qseg_next = (i0 + lane < Lq) ? sv(i0 + lane) : 0;
#pragma unroll
    for (int k = 0; k < (QCW + 63) / 64; ++k) {
      const int pc = w * QCW + 64 * k + lane;  // physical chunk
      if (64 * k + lane < QCW) {
        const int r = pc / SQ::CPR, lc = (pc % SQ::CPR) ^ (r & (SQ::CPR - 1));
        const int64_t i = min(i0 + r, Lq - 1);
        lds_dma16(qbase + i * p.qs[1] + lc * SQ::VEC, (char*)Qd + (w * QCW + 64 * k) * 16);
        lds_dma16(dobase + i * bp.dos[1] + lc * SQ::VEC, (char*)dOd + (w * QCW + 64 * k) * 16);
      }
    }
    if (p.flags) {
      // two 2048-element blocks of the saved term: forward wave block
      // (i0 % 128) / 32 of forward key tiles j0/64 and j0/64 + 1
      constexpr int CPB = 2048 * (int)sizeof(BT) / 16;
#pragma unroll
      for (int k = 0; k < BCW / 64; ++k) {
        const int pc = w * BCW + 64 * k + lane;
        const int kk = pc / CPB;
        const BT* src = biasb + bias_tile_offset(b, h, p.H, i0 / 128, j0 / 64 + kk, p.LqP, p.LkP) +
                        ((i0 % 128) / 32) * 2048 + (pc % CPB) * (16 / (int)sizeof(BT));
        lds_dma16_nt(src, (char*)Bd + (w * BCW + 64 * k) * 16);  // read once: non-temporal
      }
    }
    if (w == 0 && lane < 2 * BQ * 4 / 16) lds_dma16(rib + 2 * i0 + 4 * lane, (char*)Rd);
    if (p2c && ring) issue_ring(tw0 / 32 + qi + 4);
    if (DROP && lane < 16) lds_dma16(dropw + (int64_t)qi * NKT64 * 64 + 4 * lane, (char*)(Dd + w * 64));
  };

  // dS rows i of the wave's 32 keys: lane (g, c16) writes keys jw + 16 kk +
  // 4g + [0, 4) of query i0 + 16 mi + c16.
  typedef T vec4 __attribute__((ext_vector_type(4)));
  // dS rows i of the wave's 32 keys: lane (g, c16) writes keys jw + 8g +
  // [0, 8) of query i0 + 16 mi + c16, one 16-byte store (bf16; two for
  // fp32): NST store instructions per tile.
  typedef T vec8 __attribute__((ext_vector_type(8)));
  constexpr int NST = (BQ / 16) * (int)(sizeof(vec8) / 16);
  auto store_ds = [&](int i0, int mi, const vec8& v) {
    *reinterpret_cast<vec8*>(dsw + (int64_t)(i0 + 16 * mi + c16) * p.LkP + 8 * g) = v;
  };
  if (!any_key) {
    if (!SEGM)
      for (int qi = 0; qi < nqt; ++qi)
#pragma unroll
        for (int mi = 0; mi < BQ / 16; ++mi) store_ds(qi * BQ, mi, vec8{});
  } else {
    // K and V rows of the wave's keys stay in registers (B operands)
    frag kf[2][NS], vf[2][NS];
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) {
      const int j = jcol[jb];
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        kf[jb][s] = (j < Lk) ? M::load_contig(kbase + (int64_t)j * p.ks[1], s, g) : M::zero();
        vf[jb][s] = (j < Lk) ? M::load_contig(vbase + (int64_t)j * p.vs[1], s, g) : M::zero();
      }
    }
    {
      // zero the wave's dS^T tile (its zero columns are never written)
      vecT z;
#pragma unroll
      for (int e = 0; e < VEC; ++e) z[e] = (T)0.0f;
      static_assert(SW % VEC == 0, "whole chunks");
      for (int c = lane; c < SW / VEC; c += 64) reinterpret_cast<vecT*>(stg)[c] = z;
      // without relative terms no saved term is copied in: the bias buffers
      // hold zeros, so the scores add them unconditionally (no branch per
      // product block)
      if (!p.flags) {
        typedef uint32_t u4 __attribute__((ext_vector_type(4)));
        constexpr int NCH = BE * (int)sizeof(BT) / 16;
        for (int c = tid; c < NCH; c += 256) {
          reinterpret_cast<u4*>(Bs0)[c] = u4{0u, 0u, 0u, 0u};
          reinterpret_cast<u4*>(Bs1)[c] = u4{0u, 0u, 0u, 0u};
        }
      }
    }
    // Unmasked workgroups whose 128 keys all lie below Lk: on query tiles
    // below Lq every row is live and every pair kept, so P needs no keep
    // test per element.
    const bool keys_in = MASK == MASK_NONE && j0 + BKW <= Lk;
    // The qrgt ring holds blocks [qi, qi + 4] of the window (relative to
    // tw0 / 32) while tile qi is computed; block qi + 5 lands in the sixth
    // slot meanwhile when the next tile is qi + 1.  The first window:
    const int qfirst = SEGM ? (__builtin_amdgcn_readfirstlane(qlist[0]) & 0x3ff) : 0;
    if (p2c)
      for (int r = 0; r < 4; ++r) issue_ring(tw0 / 32 + qfirst + r);
    issue(qfirst, true, Qs0, dOs0, Bs0, Rs0, Dk0);
    lds_dma_wait();
    auto tile = [&](int n, const T* Q, const T* dO, const BT* Bt, const float* R, const uint32_t* Dw, T* nQ, T* ndO,
                    BT* nBt, float* nR, uint32_t* nDw) {
      const int ent = SEGM ? __builtin_amdgcn_readfirstlane(qlist[n]) : n;
      const int qi = ent & 0x3ff, i0 = qi * BQ;
      // This wave's copies of tile qi have landed: they were issued before
      // the previous tile's NST dS stores, its last vector-memory
      // instructions (tile 0 was waited for before the loop).
      vm_wait<NST>();
      if (MASK == MASK_SEG && w == 1 && lane < BQ) qsg[n & 1][lane] = qseg_next;
      __syncthreads();  // ... every wave's, and the previous tile is no longer read
      if (SEGM && p2c && n > 0) {
        // after skipped tiles: the blocks of this tile's window not in the
        // ring yet (their slots hold blocks no longer needed)
        const int pv = __builtin_amdgcn_readfirstlane(qlist[n - 1]) & 0x3ff;
        if (qi > pv + 1) {
          for (int x = max(qi, pv + 5); x <= qi + 4; ++x) issue_ring(tw0 / 32 + x);
          vm_wait<0>();
          __syncthreads();
        }
      }
      if (n + 1 < nlist) {
        const int qn = SEGM ? (__builtin_amdgcn_readfirstlane(qlist[n + 1]) & 0x3ff) : n + 1;
        issue(qn, qn == qi + 1, nQ, ndO, nBt, nR, nDw);
      }
      // With segments, a tile whose queries all share the workgroup's single
      // key segment needs no masking beyond the dead-row test.  Other modes:
      // tiles without a kept (query, key) pair store zeros.
      const bool full = SEGM && (ent & 0x4000);
      bool skip = !SEGM && i0 >= Lq;
      if (!skip && MASK == MASK_PAIR) {
        int keep = 0;
        const int r = tid >> 3, part = tid & 7;
        const int i = i0 + r;
        uint32_t bits = 0;
        if (i < Lq && pkb[(int64_t)i * p.pkq + i]) {
          // one 16-byte read of the mask row (rows 16-byte aligned,
          // host-checked; a 16-key chunk that starts below Lk lies in the
          // row's allocation), kept as 16 bits in LDS for the tile
          const int jb0 = j0 + part * (BKW / 8);
          if (jb0 < Lk) {
            const uint4 v = *reinterpret_cast<const uint4*>(pkb + (int64_t)i * p.pkq + jb0);
            const uint32_t wv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int q = 0; q < 16; ++q) bits |= ((wv[q >> 2] >> (8 * (q & 3))) & 0xffu) ? (1u << q) : 0u;
          }
        }
        pmask[r][part] = (uint16_t)bits;
        keep = bits != 0;
        skip = !__syncthreads_or(keep);
      }
      if (skip) {
#pragma unroll
          for (int mi = 0; mi < BQ / 16; ++mi) store_ds(i0, mi, vec8{});
        return;
      }

      // ---- scores (queries down, keys across): Q K^T + saved bias (unscaled) --------------------
      // The products run at a raised wave priority and the P / dS arithmetic
      // at the normal one, so that the SIMD's other wave fills in (dkdv
      // 158.2 -> 156.8 us in one process).
      __builtin_amdgcn_s_setprio(1);
      const float one = opaque_one();
      f32x4 sc[2][BQ / 16];
#pragma unroll
      for (int ib = 0; ib < BQ / 16; ++ib) {
        frag qa[NS];
#pragma unroll
        for (int s = 0; s < NS; ++s) qa[s] = SQ::row_frag(Q, 16 * ib + c16, s, g);
#pragma unroll
        for (int jb = 0; jb < 2; ++jb) {
          f32x4 acc = zero4();
#pragma unroll
          for (int s = 0; s < NS; ++s)
            acc = M::mma(qa[s], kf[jb][s], acc);
          {
            // rows 16*ib + 4*g + e of key column 32w + 16*jb + c16 (forward
            // tile order); without relative terms the buffer holds zeros
            const int jl = WK * w + 16 * jb;
            const int o = (jl / 64) * 2048 + ib * 1024 + ((jl % 64) / 16) * 256;
            if constexpr (sizeof(BT) == 2) {
              // one mixed-precision FMA per element adds the fp16 term
              typedef _Float16 h4 __attribute__((ext_vector_type(4)));
              const h4 v = __builtin_bit_cast(
                  h4, tr4_at(reinterpret_cast<const bf16*>(Bt) + o + (4 * g + (c16 >> 2)) * 16 + (c16 & 3) * 4));
#pragma unroll
              for (int e = 0; e < 4; ++e) acc[e] = __builtin_fmaf((float)v[e], one, acc[e]);
            } else {
              float v[4];
#pragma unroll
              for (int e = 0; e < 4; ++e) v[e] = Bt[o + (4 * g + e) * 16 + c16];
#pragma unroll
              for (int e = 0; e < 4; ++e) acc[e] += v[e];
            }
          }
          sc[jb][ib] = acc;
        }
      }

      __builtin_amdgcn_s_setprio(0);
      // ---- P, dP, dS -----------------------------------------------------------------------------
      f32x4 pp[2][BQ / 16], dsh[2][BQ / 16];
      // dropout: this lane's 16 keep bits, bit 8 ib + 4 jb + e
      uint32_t dm = 0;
      if constexpr (DROP) {
        const uint4 f4 = *reinterpret_cast<const uint4*>(Dw + w * 64 + 16 * (c16 >> 2) + 4 * g);
        const uint32_t f[4] = {f4.x, f4.y, f4.z, f4.w};
        // word e, shifted by 8 (w % 2) + c16 % 4, holds the pair (ib, jb) at
        // bit 16 ib + 4 jb: bits 0 and 4 stay, bits 16 and 20 move to 8
        // and 12, then the word's four bits go to 8 ib + 4 jb + e
        const int sh = 8 * (w & 1) + (c16 & 3);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t t = f[e] >> sh;
          dm |= ((t & 0x11u) | ((t >> 8) & 0x1100u)) << e;
        }
      }
      auto probs = [&](auto plain) {
        // segment masks: the lane's query segments, four consecutive rows
        // of each 16-row block in one 16-byte LDS read (read per element,
        // they cost segment-masked steps 4 to 13%)
        int4 qv[BQ / 16];
        if constexpr (MASK == MASK_SEG && !decltype(plain)::value) {
#pragma unroll
          for (int ib = 0; ib < BQ / 16; ++ib) qv[ib] = *reinterpret_cast<const int4*>(&qsg[n & 1][16 * ib + 4 * g]);
        }
#pragma unroll
        for (int ib = 0; ib < BQ / 16; ++ib) {
          frag dof[NS];
#pragma unroll
          for (int s = 0; s < NS; ++s) dof[s] = SQ::row_frag(dO, 16 * ib + c16, s, g);
#pragma unroll
          for (int jb = 0; jb < 2; ++jb) {
            f32x4 dp = zero4();
#pragma unroll
            for (int s = 0; s < NS; ++s)
              dp = M::mma(dof[s], vf[jb][s], dp);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int il = 16 * ib + 4 * g + e;
              const float lr = R[2 * il];
              float pe;
              if constexpr (decltype(plain)::value) {
                pe = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[jb][ib][e], sl2, -lr));
              } else {
                // rows without probabilities (dead, padding) have lr = inf and may hold an
                // unwritten saved term: they are never exponentiated
                bool keep = jkeep[jb] && lr != INFINITY;
                if (MASK == MASK_SEG && !full)
                  keep = keep && (e == 0 ? qv[ib].x : e == 1 ? qv[ib].y : e == 2 ? qv[ib].z : qv[ib].w) == jseg[jb];
                if (MASK == MASK_PAIR) keep = keep && ((pmask[il][2 * w + jb] >> c16) & 1u);
                pe = keep ? __builtin_amdgcn_exp2f(__builtin_fmaf(sc[jb][ib][e], sl2, -lr)) : 0.f;
              }
              if constexpr (DROP) {
                const bool kept = (dm >> (8 * ib + 4 * jb + e)) & 1u;
                pp[jb][ib][e] = kept ? pe : 0.f;
                dsh[jb][ib][e] = pe * ((kept ? dp[e] * p.drop_scale : 0.f) - R[2 * il + 1]);
              } else {
                pp[jb][ib][e] = pe;
                dsh[jb][ib][e] = pe * (dp[e] - R[2 * il + 1]);
              }
            }
          }
        }
      };
      // without masking: unmasked tiles inside the sequence, and segment
      // tiles listed as full (every query and key of the tile active and in
      // one segment, so every pair is kept and every row has probabilities)
      if (!DROP && ((keys_in && i0 + BQ <= Lq) || (MASK == MASK_SEG && full)))
        probs(std::true_type{});
      else
        probs(std::false_type{});
      // dS^T of the tile into the wave's LDS tile (rows j), then dS rows to
      // the workspace, four consecutive keys per lane read transposed
#pragma unroll
      for (int jb = 0; jb < 2; ++jb)
#pragma unroll
        for (int ib = 0; ib < BQ / 16; ++ib) {
          vec4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = (T)dsh[jb][ib][e];
          *reinterpret_cast<vec4*>(stg + (16 * jb + c16) * SROW + ZL + 16 * ib + 4 * g) = v;
        }
#pragma unroll
      for (int mi = 0; mi < BQ / 16; ++mi)
        store_ds(i0, mi, join_halves<T>(tr4(stg + ZL, SROW, 8 * g, 16 * mi, c16), tr4(stg + ZL, SROW, 8 * g + 4, 16 * mi, c16)));

      // ---- dV^T += dO^T P,  dK^T += Q^T dS (dO^T, Q^T read transposed) -----------------------
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int s = 0; s < BQ / M::KSTEP; ++s) {
        frag pf[2], df[2];
#pragma unroll
        for (int jb = 0; jb < 2; ++jb) {
          pf[jb] = M::from_acc(pp[jb], s);
          df[jb] = M::from_acc(dsh[jb], s);
        }
#pragma unroll
        for (int db = 0; db < ND; ++db) {
          const frag dotf = SQ::col_acc(dO, s * M::KSTEP, 16 * db, g, c16);
          const frag qtf = SQ::col_acc(Q, s * M::KSTEP, 16 * db, g, c16);
#pragma unroll
          for (int jb = 0; jb < 2; ++jb) {
            dva[db][jb] = M::mma(dotf, pf[jb], dva[db][jb]);
            dka[db][jb] = M::mma(qtf, df[jb], dka[db][jb]);
          }
        }
      }

      // ---- p2c: dK^T += qrgt[t0 + x]^T F[x] ------------------------------------------------
      if (p2c) {
        // qrgt column of x = 0 for this wave: i0 - jw - 31 + OFF (a multiple of 32)
        const int t0 = tw0 + i0 + BKW - WK - WK * w;
#pragma unroll
        for (int s = 0; s < 2 * WK / M::KSTEP; ++s) {
          frag bfr[2];
#pragma unroll
          for (int jb = 0; jb < 2; ++jb) {
            // k = x = KSTEP*s + FE*g + e  ->  staged column (i - i0) = x + (j - jw) - 31
            const int jl = 16 * jb + c16;
            const T* row = stg + jl * SROW + ZL + M::KSTEP * s + FE * g + jl - 31;
            lds_read_elems<T, FE>(bfr[jb], row);
          }
          const int t = t0 + M::KSTEP * s + FE * g;  // this lane's first k column
          const T* blk = Ring + ((t >> 5) % NRB) * RBE + ((t & 31) / VEC) * D * VEC;
#pragma unroll
          for (int db = 0; db < ND; ++db) {
            const frag af = *reinterpret_cast<const frag*>(blk + (16 * db + c16) * VEC);
#pragma unroll
            for (int jb = 0; jb < 2; ++jb) dka[db][jb] = M::mma(af, bfr[jb], dka[db][jb]);
          }
        }
      }
      __builtin_amdgcn_s_setprio(0);
    };
    for (int n = 0; n < nlist; n += 2) {
      tile(n, Qs0, dOs0, Bs0, Rs0, Dk0, Qs1, dOs1, Bs1, Rs1, Dk1);
      if (n + 1 < nlist) tile(n + 1, Qs1, dOs1, Bs1, Rs1, Dk1, Qs0, dOs0, Bs0, Rs0, Dk0);
    }
  }

  // ---- dK, dV ------------------------------------------------------------------------------
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
          vv[e] = (T)(DROP ? dva[db][jb][e] * p.drop_scale : dva[db][jb][e]);
        }
        *reinterpret_cast<vec4*>(krow + 16 * db + 4 * g) = kv;
        *reinterpret_cast<vec4*>(vrow + 16 * db + 4 * g) = vv;
      }
    }
  }
}

}  // namespace dsa
