// dsa_bwd_table.h — gradients of the projected relative tables (gfx950).
//
//   dKr[r] = s sum_{b,i,j: c(i-j)=r} dS_ij q_i,   dQr[r] = s sum_{b,i,j: p(i-j)=r} dS_ij k_j
//
// are computed per offset d = i - j first,
//   Gc[d] = sum_{b,i} dS(i, i-d) q_i,   Gp[d] = sum_{b,j} dS(j+d, j) k_j,
// and then summed onto table rows (dsa_bwd_fold_kernel): c(d) and p(d) are
// monotone in d, so the offsets of one row form a contiguous range
// (prep_segments in dsa_bwd_prep_kernel finds them).
//
// dsa_bwd_table_kernel: one workgroup = (128-offset block [d0, d0+128),
// head h, partial group: a range of the block's items).  Waves 0 and 1
// compute Gc, waves 2 and 3 Gp, each wave on its own items, staged into its
// own part of LDS (no workgroup barrier until the end).  An item is one
// batch and 32 rows:
//   Gc item: queries [i0, i0+32); region X[r][c] = dS(i0 + r, i0 - d0 - 128 + c)
//            (32 x 168); the pair (r, r + e + 1) has offset d0 + 127 - e, so
//            Gc^T[:, e] += sum_r Q^T[:, i0 + r] X[r][r + e + 1]
//   Gp item: keys [j0, j0+32); region X[rho][c] = dS(j0 + d0 + rho, j0 + c)
//            (160 x 32); the pair (c + e, c) has offset d0 + e, so
//            Gp^T[:, e] += sum_c K^T[:, j0 + c] X[c + e][c]
// Every pair of a batch with an offset in the block lies in exactly one item
// of each kind.  The B operands walk diagonals of X (one 16-bit LDS read per
// element, at compile-time offsets from a per-lane base); the k index of the
// products (the 32 rows of an item) is assigned to lane groups interleaved
// (group g holds rows 2g, 2g+1, 2g+8, 2g+9, ...), which spreads the four
// groups' diagonal reads over distinct LDS banks.  A wave keeps all 128
// offsets x D in registers (fp32) and prefetches its next item's global
// data into registers while it computes.  The two waves of a kind sum their
// accumulators through LDS and write one fp32 partial per (block, head,
// partial group, kind), with a flag; a partial whose items are all inactive
// under a mask is not written.  The Gc and Gp waves of a workgroup sweep the
// same batch's band of dS together, so the second reader of each dS line
// finds it in L2.
#pragma once

#include "dsa_bwd.h"

namespace dsa {

namespace tbcfg {
constexpr int NW = 4;
constexpr int DBW = 128;          // offsets per block
constexpr int CH = 32;            // rows of an item (Gc: queries, Gp: keys)
constexpr int XS_C = DBW + 40;    // Gc region row stride (elements; 160 columns used)
constexpr int PR = DBW + CH;      // Gp region rows (160; 159 used)
constexpr int XS_P = 40;          // Gp region row stride (elements; 32 columns used)
}  // namespace tbcfg

// k index (row of an item) of element u of a B fragment of lane group g in
// k-step s, as the sum of a per-lane part (tab_kg) and a compile-time part
// (tab_ku).  bf16: groups interleaved in pairs (rows 2g + {0,1} + 8m); fp32:
// the contiguous k-set (rows 4g + u).
template <typename T>
DSA_DEV int tab_kg(int g) {
  return sizeof(T) == 2 ? 2 * g : 4 * g;
}
template <typename T>
constexpr int tab_ku(int s, int u) {
  return sizeof(T) == 2 ? 32 * s + (u & 1) + 8 * (u >> 1) : 16 * s + u;
}

// A operand (rows of an item, transposed): lane (c16, g) gets
// R[k(s, g, u)][col0 + c16] for its k-set, R row-major with stride str.
template <typename T>
DSA_DEV typename Mfma<T>::frag tab_afrag(const T* R, int str, int s, int col0, int g, int c16) {
  if constexpr (sizeof(T) == 2) {
    // ds_read_b64_tr_b16: lane 4e + q addresses the 4-column chunk q of the
    // row that lane group g needs as its e-th k value
    const int e = c16 >> 2, q = c16 & 3;
    const int row = 32 * s + 2 * g + (e & 1) + 8 * (e >> 1);
    const T* p = R + row * str + col0 + 4 * q;
    return join8(tr4_at(p), tr4_at(p + 16 * str));
  } else {
    const int row = 16 * s + 4 * g;
    const T* p = R + row * str + col0 + c16;
    return f32x4{p[0], p[str], p[2 * str], p[3 * str]};
  }
}

// Number of 32-row items of each kind in offset block dblk and the first
// item row: Gc items start at query rows i >= max(d0, 0) and end where no key
// j = i - d < Lk is left; Gp items start at the first key with a query
// j + d >= 0 and end where no query j + d < Lq is left.
DSA_DEV void block_items(int dblk, int LkP, int Lq, int Lk, bool p2c, int* start, int* n) {
  using namespace tbcfg;
  const int d0 = -LkP + DBW * dblk;  // a multiple of 128
  int s, e;
  if (!p2c) {
    s = d0 > 0 ? d0 : 0;
    e = min(Lq, Lk + d0 + DBW - 1);
  } else {
    s = max(0, -(d0 + DBW - 1)) / CH * CH;
    e = min(Lk, Lq - d0);
  }
  *start = s;
  *n = e > s ? (e - s + CH - 1) / CH : 0;
}

// LDS of a table workgroup (a struct, so that the kernel that runs dq and
// table workgroups in one launch can overlay it with the dq kernel's).
template <typename T, int D>
struct TabLds {
  static constexpr int KSTR = D + Pad<T>::v;
  static constexpr int XELEMS =
      (tbcfg::CH * tbcfg::XS_C > tbcfg::PR * tbcfg::XS_P) ? tbcfg::CH * tbcfg::XS_C : tbcfg::PR * tbcfg::XS_P;
  static constexpr int WELEMS = XELEMS + tbcfg::CH * KSTR;  // per wave
  alignas(16) T lds[tbcfg::NW * WELEMS];
  int ilist[tbcfg::NW][64];  // per wave: the active items of a window of 64 candidates
  int nact_sh[tbcfg::NW];
};

// Workgroup blk of nblk (the logical index, whose remainder mod 8 is the
// XCD it runs on).  LISTED: a key-padding or segment mask is given
// (bp.cinfo): items without an active part are skipped and partials carry
// flags.
template <typename T, int D, bool LISTED>
DSA_DEV void table_body(const BwdParams& bp, int blk, int nblk, TabLds<T, D>& L) {
  using namespace tbcfg;
  using M = Mfma<T>;
  typedef typename M::frag frag;
  constexpr int VEC = 16 / sizeof(T);
  typedef T vecT __attribute__((ext_vector_type(VEC)));
  constexpr int ND = D / 16;
  constexpr int NEB = DBW / 16;         // 16-offset blocks
  constexpr int FE = M::FRAG_ELEMS;
  constexpr int NS = CH / M::KSTEP;     // k steps per item
  constexpr int KSTR = TabLds<T, D>::KSTR;   // item rows (Q or K) stride
  constexpr int DCH = D / VEC;               // 16-byte chunks per item row
  constexpr int XELEMS = TabLds<T, D>::XELEMS;
  constexpr int WELEMS = TabLds<T, D>::WELEMS;
  constexpr bool PREFETCH = sizeof(T) == 2;
  static_assert((XS_C * sizeof(T)) % 16 == 0 && (XS_P * sizeof(T)) % 16 == 0, "16-byte rows");
  static_assert(NW * WELEMS * sizeof(T) >= 2 * NEB * ND * 64 * 16, "LDS holds two waves' accumulators");
  const FwdParams& p = bp.f;

  T* const lds = L.lds;
  int(&ilist)[NW][64] = L.ilist;
  int* const nact_sh = L.nact_sh;

  const int tid = threadIdx.x;
  // the wave index, known to the compiler as uniform (the item loop's
  // buffer resources are then scalar)
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, g = lane >> 4, c16 = lane & 15;
  const bool p2c = w >= 2;  // wave kind: 0, 1 -> Gc; 2, 3 -> Gp
  const int sub = w & 1;
  // Work order.  Short sequences (fewer than 32 offset blocks, a grid of
  // a few workgroups per CU): blk enumerates (offset block, head,
  // partial group) with the offset blocks that have the most items first,
  // so the shortest workgroups fill in at the end of the launch.  Longer
  // ones (many workgroups per CU): the logical index (xcd_remap)
  // enumerates (head, partial group, offset block), so the offset blocks of
  // one head and group, which stage the same Q and K item rows, run on one
  // XCD side by side and share its L2 (the balance at the end matters less
  // there: 3% less time at L = 2048, 7% less at L = 4096 with documents;
  // 33% more at L = 1024 and 25% more at L = 512).
  int rank, rem;
  if (bp.NDB >= 32) {
    const int m = xcd_remap(blk, nblk);
    rank = m % bp.NDB, rem = m / bp.NDB;
  } else {
    const int per_blk = p.H * bp.NPG;
    rank = blk / per_blk, rem = blk % per_blk;
  }
  const int h = rem / bp.NPG, pg = rem % bp.NPG;
  const int mid = (bp.NDB - 1) / 2;  // central blocks hold the most pairs
  const int dblk = (rank & 1) ? mid + 1 + (rank >> 1) : mid - (rank >> 1);
  const int d0 = -p.LkP + DBW * dblk;
  const bool active = (p.flags & (p2c ? 2 : 1)) != 0;
  int rstart, nch;
  block_items(dblk, p.LkP, p.Lq, p.Lk, p2c, &rstart, &nch);
  // The block's items of one kind, (batch, 32-row chunk) batch-major, are
  // split into NPG contiguous ranges; partial group pg takes range pg.
  const int total = active ? p.B * nch : 0;
  const int per = (total + bp.NPG - 1) / bp.NPG;
  const int it_lo = min(total, pg * per), nitems = min(total, it_lo + per) - it_lo;
  // A block whose offsets all lie in the offset range of one table row of
  // its kind (where the relative position saturates, or in a wide log
  // bucket) is stored summed over its offsets, in row 0 of its partial
  // (flag 2): the fold reads one row of it instead of 128.  The fold finds
  // the same blocks from the same ranges.
  bool collapse = false;
  if (active && d0 >= -(p.Lk - 1) && d0 + DBW <= p.Lq) {
    const int R = 2 * p.A, t = p2c ? 1 : 0;
    const int r = offset_row(p.rel, d0, p.Lq, p.Lk, p.A, p2c);
    collapse = bp.rowseg[(2 * t) * R + r] <= d0 && bp.rowseg[(2 * t + 1) * R + r] >= d0 + DBW;
  }

  T* X = lds + w * WELEMS;  // this wave's region
  T* Rw = X + XELEMS;       // and its item rows (Q for Gc, K for Gp)

  f32x4 acc[NEB][ND];
#pragma unroll
  for (int eb = 0; eb < NEB; ++eb)
#pragma unroll
    for (int db = 0; db < ND; ++db) acc[eb][db] = zero4();

  // The item loop of one kind (P: Gp).
  //
  // Staging of an item, in 16-byte chunks: the region, then the item rows
  // (Q for Gc, K for Gp).  Each is a block of rows x CPR chunks walked in
  // passes of 64 / CPR rows, one chunk per lane, so a lane's byte offset
  // moves by a uniform stride from pass to pass.  The loads are buffer
  // loads whose range check returns zeros: for chunks outside the (b, h)
  // slice of dS (rows before 0 or past LqP: negative offsets are huge as
  // unsigned), for Gc chunks whose columns lie outside [0, LkP) (their
  // offset is pushed past the range), and for item rows past Lq / Lk.
  int nact = 0;  // items with an active part, this wave
  auto run = [&](auto kind) {
    constexpr bool P = decltype(kind)::value;
    constexpr int CPR = P ? CH / VEC : (DBW + CH) / VEC;  // Gc region: 160 columns read per row
    constexpr int RPI = 64 / CPR;
    constexpr int NXR = P ? PR : CH;                      // region rows
    constexpr int NP_X = (NXR + RPI - 1) / RPI;
    constexpr int RPI_R = 64 / DCH, NP_R = (CH + RPI_R - 1) / RPI_R;
    constexpr int NSLOT = NP_X + NP_R;
    constexpr int XS = P ? XS_P : XS_C;
    constexpr unsigned OOB = 0x80000000u;  // at least every range below
    const int lr = lane / CPR, lc = lane % CPR;  // region: row in pass, chunk
    const int rr = lane / DCH, rc = lane % DCH;  // item rows: row in pass, chunk
    const int64_t qks = P ? p.ks[1] : p.qs[1];
    const T* qkh = P ? (const T*)p.k + (int64_t)h * p.ks[2] : (const T*)p.q + (int64_t)h * p.qs[2];
    const int64_t qkbs = P ? p.ks[0] : p.qs[0];
    const int Lrow = P ? p.Lk : p.Lq;
    const unsigned xstride = (unsigned)(RPI * p.LkP * (int)sizeof(T));  // bytes per pass
    const unsigned rstride = (unsigned)(RPI_R * qks * (int64_t)sizeof(T));
    auto bload = [&](__amdgpu_buffer_rsrc_t rs, unsigned off) {
      return __builtin_bit_cast(vecT, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)off, 0, 0));
    };
    // Under a segment mask, dS exists only in the active tiles of 32 queries
    // x 128 keys (ChunkRange).  Bit u of an item's mask: Gc, key tile
    // kA + u of the region's columns (kA = the first); Gp, query chunk
    // cA + u of the region's rows.  Inactive parts are read as zeros and an
    // item without active parts is skipped.
    const int nqc = p.LqP / 32, nkt128 = p.LkP / 128;
    auto item_mask = [&](int b, int r0) -> int {
      if (!LISTED) return 0xff;
      const int4* ci = bp.cinfo + (int64_t)b * nqc;
      int m = 0;
      if constexpr (!P) {
        const int jc0 = r0 - d0 - DBW, kA = (jc0 >= 0 ? jc0 : jc0 - 127) / 128;
        const ChunkRange qc = chunk_range(ci, r0 / 32);
#pragma unroll
        for (int u = 0; u < 3; ++u) {
          const int k = kA + u;
          if (k >= 0 && k < nkt128 && 128 * k < jc0 + DBW + CH && qc.meets(key_tile_range(ci, k, nqc))) m |= 1 << u;
        }
      } else {
        const ChunkRange kr = key_tile_range(ci, r0 / 128, nqc);
        const int cA = (r0 + d0) / 32;  // r0 + d0 is a multiple of 32 (may be negative)
#pragma unroll
        for (int u = 0; u < PR / 32; ++u) {
          const int c = cA + u;
          if (c >= 0 && c < nqc && chunk_range(ci, c).meets(kr)) m |= 1 << u;
        }
      }
      return m;
    };
    // buffer resources and pass-0 byte offsets of item it
    struct ItemSrc {
      __amdgpu_buffer_rsrc_t xs, rs;
      unsigned xoff, roff;
      int mask;
    };
    auto item_src = [&](int it, int mask) {
      const int a = it_lo + it, b = a / nch, r0 = rstart + (a % nch) * CH;
      ItemSrc o;
      o.mask = mask;
      const T* dsb = (const T*)bp.ds + (int64_t)(b * p.H + h) * p.LqP * p.LkP;
      o.xs = __builtin_amdgcn_make_buffer_rsrc((void*)dsb, 0, p.LqP * p.LkP * (int)sizeof(T), 0x00020000);
      if constexpr (!P) {
        const int jc0 = r0 - d0 - DBW, kA = (jc0 >= 0 ? jc0 : jc0 - 127) / 128;
        const int j = jc0 + lc * VEC;  // a multiple of VEC: chunks lie wholly in or out
        const int kb = (j >= 0 ? j / 128 : 0) - kA;
        const bool ok = lr < RPI && j >= 0 && j < p.LkP && ((o.mask >> kb) & 1);
        o.xoff = ok ? (unsigned)(((r0 + lr) * p.LkP + j) * (int)sizeof(T)) : OOB;
      } else {
        o.xoff = (unsigned)(((r0 + d0 + lr) * p.LkP + r0 + lc * VEC) * (int)sizeof(T));
      }
      const T* rb = qkh + (int64_t)b * qkbs;
      o.rs = __builtin_amdgcn_make_buffer_rsrc((void*)rb, 0, (int)(((int64_t)(Lrow - 1) * qks + D) * sizeof(T)),
                                               0x00020000);
      o.roff = (unsigned)(((int64_t)(r0 + rr) * qks + rc * VEC) * sizeof(T));
      return o;
    };
    T* const xd = X + lr * XS + lc * VEC;       // LDS destinations: pass t adds t * RPI rows
    T* const rd = Rw + rr * KSTR + rc * VEC;
    auto xok = [&](int t) { return lr < RPI && lr + RPI * t < NXR; };
    auto rok = [&](int t) { return rr + RPI_R * t < CH; };

    // region offset of pass t (Gp: a pass's rows may fall in an inactive chunk)
    auto xoff_t = [&](const ItemSrc& o, int t) -> unsigned {
      if constexpr (P) {
        if (!((o.mask >> ((lr + RPI * t) >> 5)) & 1)) return OOB;
      }
      return o.xoff + t * xstride;
    };
    // list entries: item index << 8 | mask
    vecT pre[PREFETCH ? NSLOT : 1];
    auto fetch = [&](int e) {
      const ItemSrc o = item_src(e >> 8, e & 0xff);
#pragma unroll
      for (int t = 0; t < NP_X; ++t) pre[t] = bload(o.xs, xoff_t(o, t));
#pragma unroll
      for (int t = 0; t < NP_R; ++t) pre[NP_X + t] = bload(o.rs, o.roff + t * rstride);
    };
    auto commit = [&]() {
#pragma unroll
      for (int t = 0; t < NP_X; ++t)
        if (xok(t)) *reinterpret_cast<vecT*>(xd + t * RPI * XS) = pre[t];
#pragma unroll
      for (int t = 0; t < NP_R; ++t)
        if (rok(t)) *reinterpret_cast<vecT*>(rd + t * RPI_R * KSTR) = pre[NP_X + t];
    };
    auto stage_direct = [&](int e) {
      const ItemSrc o = item_src(e >> 8, e & 0xff);
      for (int t = 0; t < NP_X; ++t)
        if (xok(t)) *reinterpret_cast<vecT*>(xd + t * RPI * XS) = bload(o.xs, xoff_t(o, t));
      for (int t = 0; t < NP_R; ++t)
        if (rok(t)) *reinterpret_cast<vecT*>(rd + t * RPI_R * KSTR) = bload(o.rs, o.roff + t * rstride);
    };

    // B fragment of 16-offset block eb, k-step s: Gc reads X[k][k + e + 1],
    // Gp reads X[k + e][k], k = kg + tab_ku(s, u), e = 16 eb + c16: one
    // per-lane base and compile-time offsets
    const int kg = tab_kg<T>(g);
    const T* xb = X + (P ? c16 * XS + kg * (XS + 1) : kg * (XS + 1) + c16 + 1);
    auto bfrag = [&](int eb, int s) {
      frag f;
#pragma unroll
      for (int u = 0; u < FE; ++u) f[u] = xb[(P ? 16 * eb * XS : 16 * eb) + tab_ku<T>(s, u) * (XS + 1)];
      return f;
    };

    // The wave's items are sub, sub + 2, ...; they are taken in windows of
    // 64.  Under a mask, the items of a window with an active part are
    // listed first, each lane testing one (so the chunk summaries of a
    // window are read in one round trip).
    int* const lst = ilist[w];
    const int ncand = nitems > sub ? (nitems - sub + 1) / 2 : 0;
    for (int base = 0; base < ncand; base += 64) {
      int cnt = min(64, ncand - base);
      if (LISTED) {
        const int c = base + lane, it = sub + 2 * c;
        int m = 0;
        if (c < ncand) {
          const int a = it_lo + it;
          m = item_mask(a / nch, rstart + (a % nch) * CH);
        }
        cnt = wave_append(m != 0, (it << 8) | m, lst, 0);
        wave_lds_sync();
      }
      nact += cnt;
      auto entry = [&](int n) {
        return LISTED ? __builtin_amdgcn_readfirstlane(lst[n]) : ((sub + 2 * (base + n)) << 8) | 0xff;
      };
      if constexpr (PREFETCH) {
        if (cnt > 0) fetch(entry(0));
      }
    for (int n = 0; n < cnt; ++n) {
      if constexpr (PREFETCH) {
        commit();
        if (n + 1 < cnt) fetch(entry(n + 1));
      } else {
        stage_direct(entry(n));
      }
      wave_lds_sync();
      frag af[NS][ND];
#pragma unroll
      for (int s = 0; s < NS; ++s)
#pragma unroll
        for (int db = 0; db < ND; ++db) af[s][db] = tab_afrag<T>(Rw, KSTR, s, 16 * db, g, c16);
      // one block ahead: the next block's reads are issued before this
      // block's products (the scheduling barrier keeps the compiler from
      // hoisting more of them, which would cost registers)
      frag bcur[NS];
#pragma unroll
      for (int s = 0; s < NS; ++s) bcur[s] = bfrag(0, s);
#pragma unroll
      for (int eb = 0; eb < NEB; ++eb) {
        frag bnext[NS];
        if (eb + 1 < NEB) {
#pragma unroll
          for (int s = 0; s < NS; ++s) bnext[s] = bfrag(eb + 1, s);
        }
#pragma unroll
        for (int s = 0; s < NS; ++s)
#pragma unroll
          for (int db = 0; db < ND; ++db) acc[eb][db] = M::mma(af[s][db], bcur[s], acc[eb][db]);
        __builtin_amdgcn_sched_barrier(0);
        if (eb + 1 < NEB) {
#pragma unroll
          for (int s = 0; s < NS; ++s) bcur[s] = bnext[s];
        }
      }
      wave_lds_sync();  // the region is rewritten by the next item
    }
    }
  };
  if (p2c) run(std::true_type{});
  else run(std::false_type{});

  // Sum the two waves of each kind (1 into 0, 3 into 2) through LDS, in
  // row-major [kind][dd][d] order, then add the sums to the block's
  // accumulator (zeroed by the prep kernel) with fp32 atomics, one row of D
  // consecutive floats per wave instruction.  The workgroups of one block
  // and head meet there, so the fold reads one accumulator per block; the
  // order of the additions, and so the last bits of dKr and dQr, varies
  // from run to run.  A kind whose workgroup had no active item adds
  // nothing.  A collapsed block adds only row 0, the sum over its offsets.
  constexpr int RS = D + 4;  // fp32 row stride of the sums in LDS
  static_assert(NW * WELEMS * sizeof(T) >= 2 * DBW * RS * sizeof(float), "LDS holds both kinds' sums");
  if (lane == 0) nact_sh[w] = nact;
  __syncthreads();  // every wave is done with its region
  const bool any = nact + nact_sh[w ^ 1] > 0;
  float* red = reinterpret_cast<float*>(lds) + (p2c ? DBW * RS : 0);
  auto put = [&](bool add) {
#pragma unroll
    for (int eb = 0; eb < NEB; ++eb) {
      const int e = 16 * eb + c16;
      const int dd = p2c ? e : DBW - 1 - e;  // offset d0 + dd
#pragma unroll
      for (int db = 0; db < ND; ++db) {
        f32x4* r = reinterpret_cast<f32x4*>(red + dd * RS + 16 * db + 4 * g);
        *r = add ? *r + acc[eb][db] : acc[eb][db];
      }
    }
  };
  if (sub == 1) put(false);
  __syncthreads();
  if (sub == 0) put(true);
  __syncthreads();
  if (active && any) {
    float* out = bp.gpart + ((int64_t)(h * bp.NDB + dblk) * 2 + (p2c ? 1 : 0)) * DBW * D;
    const int tt = sub * 64 + lane;  // 128 threads of this kind
    if (collapse) {
      if (tt < D) {
        float sum = 0.f;
        for (int dd = 0; dd < DBW; ++dd) sum += red[dd * RS + tt];
        unsafeAtomicAdd(out + tt, sum);
      }
    } else {
#pragma unroll 8
      for (int i = 0; i < DBW * D / 128; ++i) {
        const int f = 128 * i + tt, dd = f / D, d = f % D;
        unsafeAtomicAdd(out + f, red[dd * RS + d]);
      }
    }
  }
}

template <typename T, int D, bool LISTED>
__global__ __launch_bounds__(256, 2) void dsa_bwd_table_kernel(BwdParams bp) {
  __shared__ TabLds<T, D> L;
  table_body<T, D, LISTED>(bp, blockIdx.x, gridDim.x, L);
}

// tab[h][r][:] (+)= s * sum over offsets d with row(d) = r of the block
// accumulators (accumulated into fp32, or written in fp32 or bf16).  WPR
// waves per (table, h, r), 256 / (64 WPR) rows per workgroup: the WPR * 64
// / (D/4) parts of a row split the units of its offset range [begin, end)
// (from prep_segments), each part with four independent sums so that four
// loads are in flight; lanes of a part hold 4 columns each.  The parts are
// summed with lane shuffles and, across waves, through LDS in a fixed
// order.  Long sequences use WPR = 4: the rows where the relative position
// saturates then hold thousands of offsets; short ones one wave a row, four
// rows a workgroup (a quarter of the workgroups to launch).
template <int D, int WPR>
__global__ __launch_bounds__(256) void dsa_bwd_fold_kernel(BwdParams bp) {
  using namespace tbcfg;
  const FwdParams& p = bp.f;
  const int R = 2 * p.A;
  constexpr int NT = 64 * WPR;  // threads of one row
  constexpr int Q4 = D / 4, NP = NT / Q4, NWV = WPR;
  const int unit = blockIdx.x * (4 / WPR) + (int)(threadIdx.x / NT);
  if (unit >= 2 * p.H * R) return;  // uniform over a row's waves
  const int t = unit / (p.H * R), h = (unit / R) % p.H, r = unit % R;
  if (!(p.flags & (1 << t))) return;
  const bool q = t == 1;  // false: dKr (c2p), true: dQr (p2c)
  const int c4 = threadIdx.x % Q4, part = (threadIdx.x % NT) / Q4;
  const int beg = bp.rowseg[(2 * t) * R + r], end = bp.rowseg[(2 * t + 1) * R + r];
  // The range splits into single offsets at its ends and whole offset
  // blocks between them (stored summed by the table kernel, row 0).
  const int LkP = p.LkP;
  const int b1 = beg + (DBW - (beg + LkP) % DBW) % DBW, b2 = end - (end + LkP) % DBW;  // beg + LkP > 0
  int nl = end - beg, nf = 0, nr = 0;
  if (b2 - b1 >= DBW) {
    nl = b1 - beg;
    nf = (b2 - b1) / DBW;
    nr = end - b2;
  }
  const int npairs = nl + nf + nr;
  // accumulator row of unit it (a single offset, or a whole block's row 0)
  auto pair_val = [&](int it) {
    const bool whole = it >= nl && it < nl + nf;
    const int d = it < nl ? beg + it : whole ? b1 + (it - nl) * DBW : b2 + (it - nl - nf);
    const int dblk = (d + LkP) / DBW, dd = whole ? 0 : (d + LkP) % DBW;
    return *reinterpret_cast<const f32x4*>(bp.gpart + ((int64_t)(h * bp.NDB + dblk) * 2 + t) * DBW * D +
                                           (int64_t)dd * D + 4 * c4);
  };
  f32x4 a4[4] = {zero4(), zero4(), zero4(), zero4()};
  int it = part;
  for (; it + 3 * NP < npairs; it += 4 * NP) {
#pragma unroll
    for (int u = 0; u < 4; ++u) a4[u] += pair_val(it + u * NP);
  }
  for (; it < npairs; it += NP) a4[0] += pair_val(it);
  f32x4 acc = (a4[0] + a4[1]) + (a4[2] + a4[3]);
#pragma unroll
  for (int m = Q4; m < 64; m <<= 1)
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] += __shfl_xor(acc[e], m);
  if constexpr (NWV > 1) {
    __shared__ f32x4 wsum[NWV][Q4];
    const int w = threadIdx.x / 64, lane = threadIdx.x % 64;
    if (lane < Q4) wsum[w][lane] = acc;
    __syncthreads();
    if (w != 0) return;
    acc = wsum[0][c4];
#pragma unroll
    for (int k = 1; k < NWV; ++k) acc += wsum[k][c4];
  }
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
