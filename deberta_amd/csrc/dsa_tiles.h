// dsa_tiles.h — building blocks shared by the forward and the backward
// kernels: parameter blocks, tile loaders and the relative terms of the
// disentangled score
//     s(i, j) = q_i.k_j + q_i.Kr[c(i-j)] + k_j.Qr[p(i-j)]
// (deberta_v2_native.py:604 and the c2p/p2c terms of :389-410).
#pragma once

#include <type_traits>

#include "dsa_common.h"

namespace dsa {

struct FwdParams {
  const void* q;
  const void* k;
  const void* v;
  const void* kr;
  const void* qr;
  const int32_t* rel;
  const uint8_t* kk;
  const uint8_t* pk;
  const int32_t* seg;   // segment ids [B, L] (0: inactive token) or null
  void* out;
  float* lse;
  void* bias;       // saved relative term [B, H, LqP, LkP] or null
  const int* order; // launch order of the (batch row, tile) items, heaviest first, or null (dsa_order.h)
  const void* qc;   // query rows of the c2p term [B, Lq, H, D] (carries p2p), or null: q
  int64_t qs[3], ks[3], vs[3], os[3], qcs[3];
  int64_t krs[2], qrs[2];           // kr / qr element strides of head and table row
  int64_t krk, qrk;                 // element stride between the 64-byte k-steps of a table row
  int64_t kkb, pkb, pkq, pkh, segb;  // pkh: head stride of a per-head pair mask (0: shared)
  int B, H, Lq, Lk, A, flags;
  int LqP, LkP;     // Lq, Lk rounded up to 128 (extents of bias and dS^T)
  float scale;
  // attention dropout: the keep bits (dsa_dropout.h) and the scale of the
  // kept probabilities, 65536 / (65536 - t); null without dropout
  const uint32_t* drop;
  float drop_scale;
  void* olo;        // bf16 only: O's rounding residual, with out's strides, or null
};

struct BwdParams {
  FwdParams f;
  const void* dout;
  int64_t dos[3];
  void* dq;
  void* dk;
  void* dv;
  int64_t dqs[3], dks[3], dvs[3];
  void* dqc;        // with f.qc: the c2p part of dq, written here instead of into dq
  int64_t dqcs[3];
  void* dkr;        // table gradients: fp32 accumulated, or fp32 / bf16 overwritten
  void* dqr;
  int dtab_bf16, dtab_overwrite;
  // workspace
  float* rowinfo;   // [B, H, LqP, 2]: lse*log2e (inf: dead or padding row), dO . O
  void* ds;         // dS [B, H, f.LqP, f.LkP] (rows = queries), zero outside [0, Lq) x [0, Lk)
  void* krgt;       // [H, D, TGP]: krgt[h][d][t] = Kr[h][c(t - OFF)][d]
  void* qrgt;       // [H, D, TGP]: qrgt[h][d][t] = Qr[h][p(t - OFF)][d]
  float* gpart;     // table-gradient block accumulators [H][NDB][2][128][D], fp32: zeroed by the prep
                    // kernel, added to by the table kernel (a block summed over its offsets: row 0)
  int* rowseg;      // [2][2][R]: offsets [begin, end) of each table row (c2p, p2c)
  int4* cinfo;      // segment masks: [B][LqP / 32] per 32-token chunk (lo, hi, all active, 0)
  const int* korder;  // dkdv launch order of the (batch row, key tile) items, or null (dsa_order.h)
  const int* qorder;  // dq launch order of the (batch row, query tile) items, or null
  int TGP, OFF;     // row length and offset origin of krgt / qrgt
  int NDB, NPG;     // offset blocks, partial groups per block (item ranges)
};

// Segment view of the key-padding (MASK_KEY) and segment-id (MASK_SEG)
// masks: token i of batch row b belongs to segment seg(i), 0 meaning an
// inactive token.  Pair (i, j) is kept iff seg(i) != 0 and seg(i) ==
// seg(j), and a query with seg 0 is a dead row.  A key-padding mask is the
// case seg = (keep ? 1 : 0): a live query keeps exactly the kept keys.  The
// reference's document-block mask (training/compile.py:310-349) is the case
// seg = document id: its pad queries are dead rows, whose single kept key
// (the CLS edge) never reaches an output.
constexpr bool seg_mode(int mask) { return mask == MASK_KEY || mask == MASK_SEG; }

template <int MASK>
struct SegView {
  const uint8_t* kk;
  const int32_t* sg;
  DSA_DEV SegView(const FwdParams& p, int b)
      : kk(MASK == MASK_KEY ? p.kk + (int64_t)b * p.kkb : nullptr),
        sg(MASK == MASK_SEG ? p.seg + (int64_t)b * p.segb : nullptr) {}
  DSA_DEV int operator()(int i) const {
    if constexpr (MASK == MASK_KEY) return kk[i] != 0;
    else return sg[i];
  }
};

// The same view chosen at run time (kernels not specialised on the mask).
DSA_DEV int seg_at(const FwdParams& p, int b, int i) {
  return p.seg ? p.seg[(int64_t)b * p.segb + i] : (p.kk[(int64_t)b * p.kkb + i] != 0);
}

// Backward tile activity under a segment mask, from the per-chunk summaries
// (dsa_bwd_prep_kernel): the dkdv kernel computes the dS tile of query chunk
// c (32 queries) and key tile k (128 keys) iff the chunk's segment range
// meets the union of the key tile's four chunk ranges, and writes nothing
// for other tiles; the dq and table kernels read dS only where this
// predicate holds (zeros elsewhere), so all three agree on every element.
// The dS of a pair outside an active tile is zero: the tile holds no pair of
// one segment.
struct ChunkRange {
  int lo, hi, all;
  DSA_DEV bool meets(const ChunkRange& o) const { return lo <= hi && o.lo <= o.hi && lo <= o.hi && o.lo <= hi; }
};
DSA_DEV ChunkRange chunk_range(const int4* ci, int c) {
  const int4 v = ci[c];
  return ChunkRange{v.x, v.y, v.z};
}
// union of the ranges of key tile k's four chunks (chunks past nchunks are
// empty)
DSA_DEV ChunkRange key_tile_range(const int4* ci, int k, int nchunks) {
  ChunkRange r{0x7fffffff, (int)0x80000000, 1};
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int c = 4 * k + u;
    if (c < nchunks) {
      const ChunkRange x = chunk_range(ci, c);
      r.lo = min(r.lo, x.lo);
      r.hi = max(r.hi, x.hi);
      r.all = r.all && x.all;
    } else {
      r.all = 0;
    }
  }
  return r;
}

// Range [lo, hi] of the nonzero segments among a set of tokens (lo > hi if
// none) and whether every token of the set is active.  Every thread of the
// workgroup calls it (it holds two barriers); threads with has = false
// contribute nothing.  red: NW * 3 ints of LDS.
struct SegRange {
  int lo, hi;
  bool all;
  DSA_DEV bool any() const { return lo <= hi; }
  DSA_DEV bool meets(int s) const { return s != 0 && s >= lo && s <= hi; }
};
DSA_DEV SegRange wg_seg_range(int s, bool has, int* red) {
  constexpr int NWG = 4;
  const bool act = has && s != 0;
  int lo = wave_min(act ? s : 0x7fffffff), hi = wave_max(act ? s : (int)0x80000000);
  const int all = wave_and((!has || s != 0) ? 1 : 0);
  const int w = threadIdx.x >> 6;
  __syncthreads();  // red may still be read by an earlier call
  if ((threadIdx.x & 63) == 0) {
    red[3 * w] = lo;
    red[3 * w + 1] = hi;
    red[3 * w + 2] = all;
  }
  __syncthreads();
  SegRange r{0x7fffffff, (int)0x80000000, true};
#pragma unroll
  for (int k = 0; k < NWG; ++k) {
    r.lo = min(r.lo, red[3 * k]);
    r.hi = max(r.hi, red[3 * k + 1]);
    r.all = r.all && red[3 * k + 2] != 0;
  }
  return r;
}

template <typename T>
struct Pad {
  static constexpr int v = 16 / sizeof(T);  // one 16-byte pad per LDS row
};

// Copies rows [row0, row0 + ROWS) of a [L, D] strided matrix into LDS
// (row-major, stride `str`), zero-filling rows >= nvalid.  If `dstT` is
// given the tile is also stored transposed ([D][strT]).
template <typename T, int D, int ROWS, int NT>
DSA_DEV void load_rows(T* dst, int str, T* dstT, int strT, const T* src, int64_t rs, int row0, int nvalid,
                       int tid) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int CPR = D / VEC;
  typedef T vecT __attribute__((ext_vector_type(VEC)));
  for (int c = tid; c < ROWS * CPR; c += NT) {
    const int r = c / CPR;
    const int d0 = (c % CPR) * VEC;
    vecT x;
    if (row0 + r < nvalid) {
      x = *reinterpret_cast<const vecT*>(src + (int64_t)(row0 + r) * rs + d0);
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) x[e] = (T)0.0f;
    }
    if (dst) *reinterpret_cast<vecT*>(dst + r * str + d0) = x;
    if (dstT) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) dstT[(d0 + e) * strT + r] = x[e];
    }
  }
}

// ---------------------------------------------------------------------------
// Offset-indexed ("delta") bands.
//
// For a 128-query x 64-key tile the offsets i - j span a window of 191
// values; x = (i - i0) - (j - j0) + 63 indexes it.  Instead of computing the
// relative products per table row and looking the row up per score element,
// the bands are computed per offset: row x of the c2p band is
// q_i . Kr[c(x)], row x of the p2c band is k_j . Qr[p(x)], with the table
// rows gathered when the MFMA operands are loaded.  The score element (i, j)
// then reads band row x(i, j), whose LDS offset is a compile-time constant
// plus a per-lane base: no per-element table lookups or bounds checks.
//   c2p: per wave, rows x in [32w, 32w + 96) x the wave's 32 queries
//   p2c: per workgroup, rows x in [0, 192) x the 64 keys, shared by all waves
// Band values are stored unscaled, in fp16 for bf16 inputs (saturated to the
// fp16 range) and in fp32 for fp32 inputs; the gather adds them to the
// unscaled score (one mixed-precision FMA).
// ---------------------------------------------------------------------------
template <typename T>
struct BandType {
  typedef float type;
};
template <>
struct BandType<bf16> {
  typedef _Float16 type;
};

namespace dcfg {
constexpr int WQ = 32;          // queries per wave
constexpr int BK = 64;          // keys per tile
constexpr int NW = 4;           // waves per workgroup
constexpr int BQ = NW * WQ;     // queries per workgroup
constexpr int XW = WQ + BK;     // c2p band rows per wave (95 used)
constexpr int XG = BQ + BK;     // p2c band rows per workgroup (191 used)
// c2p band, stored per query (row i, offsets x contiguous) so that a lane's
// four MFMA results are one write; the stride puts 16 rows' 8-byte chunks
// in distinct banks
constexpr int CTS = 104;
// p2c band, stored per offset (row x, the 64 keys contiguous) so that a
// lane's four MFMA results (four consecutive keys) are two 4-byte writes;
// the odd dword stride (33 for fp16) spreads the gather's 16 consecutive
// offsets over distinct banks
constexpr int PBT = BK + 2;
constexpr int CB_ELEMS = WQ * CTS;
constexpr int PB_ELEMS = XG * PBT;
}  // namespace dcfg

// The relative tables re-laid by k-step for the forward's band loads:
// element d of row r of head h at ((h * NS + d / KS) * R + r) * KS + d % KS,
// KS the elements of 64 bytes and NS = D / KS.  The k-step of 16
// consecutive table rows that one load instruction of the bands gathers is
// then 1 KB of contiguous memory (8 cache lines; the rows of consecutive
// offsets are consecutive or repeated) instead of 16 row segments in 16
// lines.  One thread per 16 bytes; blockIdx.y = table (0: kr, 1: qr).
struct TableKs {
  const void* src[2];
  int64_t hs[2], rs[2];  // source element strides of head and row
  void* dst[2];
  int H, R, D, esize;
};
// Block bx of table tb's copy (256 16-byte chunks).
DSA_DEV void table_ks_block(const TableKs& t, int bx, int tb) {
  if (!t.src[tb]) return;
  const int per16 = 16 / t.esize, ks = 64 / t.esize, ns = t.D / ks;
  const int64_t n = (int64_t)t.H * ns * t.R * (ks / per16);
  const int64_t c = (int64_t)bx * 256 + threadIdx.x;
  if (c >= n) return;
  const int q = (int)(c % (ks / per16));
  int64_t rest = c / (ks / per16);
  const int r = (int)(rest % t.R);
  rest /= t.R;
  const int s = (int)(rest % ns), h = (int)(rest / ns);
  const char* src = (const char*)t.src[tb] + ((int64_t)h * t.hs[tb] + (int64_t)r * t.rs[tb] + s * ks + q * per16) * t.esize;
  *reinterpret_cast<uint4*>((char*)t.dst[tb] + c * 16) = *reinterpret_cast<const uint4*>(src);
}
__global__ __launch_bounds__(256) void dsa_table_ks_kernel(TableKs t) { table_ks_block(t, blockIdx.x, blockIdx.y); }

// Row tables of one tile: crow[x] / prow[x] are the element offsets (row *
// row stride) of the c2p / p2c table rows of offset x (x = (i - i0) - (j -
// j0) + 63, i0 / j0 the tile's first query / key), for x in [0, 192); the
// host checks that they fit in 32 bits.
// rel_of_tile reads thread tid's relative position (tid < XG), store_row_tables
// turns it into the two row offsets.
DSA_DEV int rel_of_tile(const int32_t* rel, int i0, int j0, int Lq, int Lk, int tid) {
  int d = i0 - j0 - (dcfg::BK - 1) + tid;
  d = min(max(d, -(Lk - 1)), Lq - 1);
  return rel[d + Lk - 1];
}

DSA_DEV void store_row_tables(int* crow, int* prow, int t, int A, int krs, int qrs, int tid) {
  if (tid < dcfg::XG) {
    t = min(max(t, -A), A);
    crow[tid] = c2p_row(t, A) * krs;
    prow[tid] = p2c_row(t, A) * qrs;
  }
}

// The saved relative term (dsa_fwd_args.bias) is stored per forward tile of
// 128 queries x 64 keys, 8192 elements in the order in which the forward's
// lanes hold them, so every store instruction writes 512 contiguous bytes:
//   element (i, j) of tile (i / 128, j / 64) is at
//   ((((w * 2 + ib) * 4 + jb) * 16 + c16) * 4 + g) * 4 + e
// with w = i % 128 / 32, ib = i % 32 / 16, c16 = i % 16, jb = j % 64 / 16,
// g = j % 16 / 4, e = j % 4.  Offset of the first element of a tile:
DSA_DEV int64_t bias_tile_offset(int b, int h, int H, int qt, int kt, int LqP, int LkP) {
  return (((int64_t)(b * H + h) * (LqP / 128) + qt) * (LkP / 64) + kt) * 8192;
}

// Stores four values at p[0..3] as two halves of two elements (p only
// 4-byte aligned for fp16, 8-byte aligned for fp32).  fp16 values are
// converted two at a time with round-toward-zero, which also saturates: a
// finite value never rounds to infinity.
template <typename B>
DSA_DEV void store4_halves(B* p, const f32x4& v) {
  if constexpr (sizeof(B) == 2) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    *reinterpret_cast<h2*>(p) = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_pkrtz(v[0], v[1]));
    *reinterpret_cast<h2*>(p + 2) = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_pkrtz(v[2], v[3]));
  } else {
    typedef float f2 __attribute__((ext_vector_type(2)));
    *reinterpret_cast<f2*>(p) = f2{v[0], v[1]};
    *reinterpret_cast<f2*>(p + 2) = f2{v[2], v[3]};
  }
}

// Stores four values at p[0..3] (fp16: round-toward-zero pair conversion,
// saturating as in store4_halves).
template <typename B>
DSA_DEV void store4_contig(B* p, const f32x4& v) {
  if constexpr (sizeof(B) == 2) {
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 a = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_pkrtz(v[0], v[1]));
    const h2 c = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_pkrtz(v[2], v[3]));
    *reinterpret_cast<h4*>(p) = h4{a[0], a[1], c[0], c[1]};
  } else {
    *reinterpret_cast<f32x4*>(p) = v;
  }
}

// Adds the c2p + p2c terms to a transposed score tile (keys down,
// queries across; y[ib][jb][e] = key 16*jb + 4*g + e, query 32*w + 16*ib +
// c16 of the tile).  y holds q.k on entry and q.k + c2p + p2c (unscaled)
// on return.
//   kf: A fragments of the 64 key rows, qf: B fragments of the wave's queries
//   (the c2p term's query rows: q, or qc when it is given)
//   cb: this wave's c2p band (WQ * CTS), pb: the shared p2c band (XG * PBT)
//   crow, prow: the tile's table row offsets (store_row_tables)
//   krk, qrk: element strides between the 64-byte k-steps of a table row
//   GR: c2p row blocks whose table rows are loaded before their products
//       (all six: one L2 round trip per tile instead of six)
//   bias: if not null, where this lane's part of the tile's saved relative
//         term goes (see bias_tile_offset): the unscaled c2p + p2c values,
//         stored for the backward
// In two parts, so that a caller can issue loads between them:
// band_products_T computes both bands into LDS (its table-row loads are all
// waited for on return), band_gather_T (which begins with a __syncthreads:
// the p2c band is shared) adds them to y and stores the saved term.  Call
// both from every thread of the workgroup.
template <typename T, int D, int GR>
DSA_DEV void band_products_T(const typename Mfma<T>::frag (&kf)[4][D / Mfma<T>::KSTEP],
                             const typename Mfma<T>::frag (&qf)[2][D / Mfma<T>::KSTEP],
                             typename BandType<T>::type* cb, typename BandType<T>::type* pb, const int* crow,
                             const int* prow, int w, int g, int c16, const T* krh, const T* qrh, int64_t krk,
                             int64_t qrk, int flags) {
  using M = Mfma<T>;
  typedef typename M::frag frag;
  typedef typename BandType<T>::type BT;
  using namespace dcfg;
  constexpr int NS = D / M::KSTEP;
  constexpr int FE = M::FRAG_ELEMS;
  // k-step s of a table row: FE elements of lane group g at rowp + s * krk + FE * g
  auto row_frag = [&](const T* rowp, int64_t ks, int s) {
    return *reinterpret_cast<const frag*>(rowp + s * ks + FE * g);
  };
  if (flags & 1) {
    // GR row blocks have their table rows requested together (one L2
    // round trip per group)
    static_assert((XW / 16) % GR == 0, "whole groups");
#pragma unroll
    for (int rb0 = 0; rb0 < XW / 16; rb0 += GR) {
      frag af[GR][NS];
#pragma unroll
      for (int u = 0; u < GR; ++u) {
        const T* rowp = krh + crow[WQ * w + 16 * (rb0 + u) + c16];
#pragma unroll
        for (int s = 0; s < NS; ++s) af[u][s] = row_frag(rowp, krk, s);
      }
#pragma unroll
      for (int u = 0; u < GR; ++u)
#pragma unroll
        for (int ib = 0; ib < 2; ++ib) {
          f32x4 acc = zero4();
#pragma unroll
          for (int s = 0; s < NS; ++s) acc = M::mma(af[u][s], qf[ib][s], acc);
          store4_contig<BT>(cb + (16 * ib + c16) * CTS + 16 * (rb0 + u) + 4 * g, acc);
        }
    }
  }
  if (flags & 2) {
#pragma unroll
    for (int t = 0; t < XG / 16 / NW; ++t) {
      const int xb = w + NW * t;
      const T* rowp = qrh + prow[16 * xb + c16];
      frag bf[NS];
#pragma unroll
      for (int s = 0; s < NS; ++s) bf[s] = row_frag(rowp, qrk, s);
#pragma unroll
      for (int jb = 0; jb < 4; ++jb) {
        f32x4 acc = zero4();
#pragma unroll
        for (int s = 0; s < NS; ++s) acc = M::mma(kf[jb][s], bf[s], acc);
        store4_halves<BT>(pb + (16 * xb + c16) * PBT + 16 * jb + 4 * g, acc);
      }
    }
  }
}

template <typename T, int D>
DSA_DEV void band_gather_T(f32x4 (&y)[2][4], const typename BandType<T>::type* cb,
                           const typename BandType<T>::type* pb, int w, int g, int c16, int flags,
                           typename BandType<T>::type* bias) {
  typedef typename BandType<T>::type BT;
  using namespace dcfg;
  __syncthreads();
  // c2p: x - 32w = (16*ib + c16) - (16*jb + 4*g + e) + 63; the four e are
  // consecutive x (descending) of one query row
  const BT* cbase = cb + c16 * CTS + c16 - 4 * g + 60;
  // p2c: row x = 32w + (16*ib + c16) - (16*jb + 4*g + e) + 63, key 16*jb + 4*g + e
  const BT* pbase = pb + (WQ * w + c16 - 4 * g + 63) * PBT + 4 * g;
  // The two terms are summed in the band type (for fp16: one rounding of the
  // exact sum, which is also the value saved), then added to the score with
  // one mixed-precision FMA per element.  The uniform flag test sits
  // outside the loops.
  const float one = opaque_one();
  // c2p reads of a 16-bit band: the four elements at cbase + K (K a
  // multiple of 16, so every read shares cbase's alignment) lie in three
  // dwords from (cbase & ~3) + K; one byte selector per lane (by that
  // alignment) picks the pairs (e = 0, 1) and (e = 2, 3) of bs below, which
  // run down the band row (x descending), with one v_perm_b32 each.
  typedef const __attribute__((address_space(3))) unsigned* lds_u32;
  // (The base is moved 48 elements down, which keeps its alignment, so that
  // every block's dword offset is non-negative: an immediate of the read.)
  const lds_u32 cq = (lds_u32)((uintptr_t)(cbase - 48) & ~(uintptr_t)3);
  const unsigned csel = ((uintptr_t)cbase & 2) ? 0x03020504u : 0x01000302u;
  // Whether the term is saved is uniform (one pointer for the workgroup):
  // the gather is compiled with and without the stores, so that no branch
  // splits its eight blocks.
  const bool save = __builtin_amdgcn_readfirstlane(bias != nullptr ? 1 : 0) != 0;
  auto gather = [&](auto with_c, auto with_p, auto with_s) {
    typedef BT b4 __attribute__((ext_vector_type(4)));
    typedef BT b2 __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int ib = 0; ib < 2; ++ib)
#pragma unroll
      for (int jb = 0; jb < 4; ++jb) {
        BT bs[4];
        bool done = false;
        if constexpr (sizeof(BT) == 2) {
          if constexpr (decltype(with_c)::value) {
            const int kd = (16 * ib * CTS + 16 * (ib - jb) + 48) / 2;
            const unsigned d0 = cq[kd], d1 = cq[kd + 1], d2 = cq[kd + 2];
            b2 hi = __builtin_bit_cast(b2, __builtin_amdgcn_perm(d2, d1, csel));  // elements 3, 2
            b2 lo = __builtin_bit_cast(b2, __builtin_amdgcn_perm(d1, d0, csel));  // elements 1, 0
            if constexpr (decltype(with_p)::value) {
              hi = hi + b2{pbase[(16 * ib - 16 * jb) * PBT + 16 * jb], pbase[(16 * ib - 16 * jb - 1) * PBT + 16 * jb + 1]};
              lo = lo + b2{pbase[(16 * ib - 16 * jb - 2) * PBT + 16 * jb + 2],
                           pbase[(16 * ib - 16 * jb - 3) * PBT + 16 * jb + 3]};
            }
            bs[0] = hi[0], bs[1] = hi[1], bs[2] = lo[0], bs[3] = lo[1];
            done = true;
          }
        }
        if (!done) {
          b4 cv;
          if constexpr (decltype(with_c)::value) lds_read_elems<BT, 4>(cv, cbase + 16 * ib * CTS + 16 * (ib - jb));
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const BT pv = decltype(with_p)::value ? pbase[(16 * ib - 16 * jb - e) * PBT + 16 * jb + e] : (BT)0.0f;
            if constexpr (decltype(with_c)::value) bs[e] = decltype(with_p)::value ? cv[3 - e] + pv : cv[3 - e];
            else bs[e] = pv;
          }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) y[ib][jb][e] = __builtin_fmaf((float)bs[e], one, y[ib][jb][e]);
        // Non-temporal stores: the saved term (201 MB at B=32, L=512) is
        // read only by the backward.  Forwards run back to back (the layers
        // of a model) take 123 against 144 us at the headline shape with
        // them (ordinary stores leave the previous forward's term to be
        // written back from the caches meanwhile); one layer's forward
        // followed by its backward takes the same time either way.
        if constexpr (decltype(with_s)::value)
          __builtin_nontemporal_store(b4{bs[0], bs[1], bs[2], bs[3]}, reinterpret_cast<b4*>(bias + (ib * 4 + jb) * 256));
      }
  };
  using yes = std::true_type;
  using no = std::false_type;
  if ((flags & 3) == 3) {
    if (save) gather(yes{}, yes{}, yes{});
    else gather(yes{}, yes{}, no{});
  } else if (flags & 1) {
    if (save) gather(yes{}, no{}, yes{});
    else gather(yes{}, no{}, no{});
  } else {
    if (save) gather(no{}, yes{}, yes{});
    else gather(no{}, yes{}, no{});
  }
}

template <typename T, int D, int GR>
DSA_DEV void add_delta_bands_T(f32x4 (&y)[2][4], const typename Mfma<T>::frag (&kf)[4][D / Mfma<T>::KSTEP],
                               const typename Mfma<T>::frag (&qf)[2][D / Mfma<T>::KSTEP],
                               typename BandType<T>::type* cb, typename BandType<T>::type* pb, const int* crow,
                               const int* prow, int w, int g, int c16, const T* krh, const T* qrh, int64_t krk,
                               int64_t qrk, int flags, typename BandType<T>::type* bias = nullptr) {
  band_products_T<T, D, GR>(kf, qf, cb, pb, crow, prow, w, g, c16, krh, qrh, krk, qrk, flags);
  band_gather_T<T, D>(y, cb, pb, w, g, c16, flags, bias);
}

}  // namespace dsa
