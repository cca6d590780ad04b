// dsa_capi.hip — C ABI of libdsa.so (declared in include/dsa.h): argument
// validation, kernel selection and launches for the fused disentangled
// attention.  Every launch goes on the caller's stream.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <type_traits>
#include <string>

#include "../../include/dsa.h"
#include "../../include/dsa_block.h"
#include "dsa_bias.h"
#include "dsa_bwd.h"
#include "dsa_bwd_dkdv.h"
#include "dsa_bwd_dq.h"
#include "dsa_bwd_dqtab.h"
#include "dsa_bwd_table.h"
#include "dsa_dropout.h"
#include "dsa_order.h"
#include "dsa_fwd.h"
#include "dsa_rows.h"

// Library-owned scratch of dsa_fwd_static: the launch order's cost and
// order arrays for up to 65536 (batch row, query tile) items, 512 KiB, one
// copy per GPU for the life of the process.  Host code never uses the
// array's name as an address: static_scratch_locked() resolves this GPU's
// copy (hipGetSymbolAddress with that device current) and keeps it once the
// lookup has succeeded.
constexpr size_t kStaticScratchBytes = 512 * 1024;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

namespace {

thread_local std::string g_err;

int fail(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
int fail(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return 1;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

int round_up(int x, int a) { return (x + a - 1) / a * a; }

int elem_bytes(int dtype) { return dtype == DSA_BF16 ? 2 : 4; }

// The c2p term's query rows (qc, optional): c2p on, aligned like q.
int check_qc(const dsa_fwd_args* a) {
  if (!a->qc) return 0;
  if (!(a->flags & DSA_C2P)) return fail("dsa: qc (the c2p term's query rows) needs DSA_C2P and kr");
  const int vec = 16 / elem_bytes(a->dtype);
  if (!aligned16(a->qc)) return fail("dsa: qc must be 16-byte aligned");
  for (int s = 0; s < 3; ++s)
    if (a->qc_strides[s] % vec != 0) return fail("dsa: qc strides must be multiples of %d elements", vec);
  return 0;
}

// Checks shared by forward and backward.  Shapes are validated on the host
// so every access the kernels make stays inside the caller's buffers.
int check_fwd(const dsa_fwd_args* a) {
  if (!a) return fail("dsa: null arguments");
  if (a->dtype != DSA_BF16 && a->dtype != DSA_F32) return fail("dsa: unsupported dtype %d", a->dtype);
  if (a->D != 32 && a->D != 64) return fail("dsa: head dim must be 32 or 64, got %d", a->D);
  if (a->B < 1 || a->H < 1 || a->Lq < 1 || a->Lk < 1)
    return fail("dsa: empty shape B=%d H=%d Lq=%d Lk=%d", a->B, a->H, a->Lq, a->Lk);
  if (a->B > 65535 || a->H > 65535) return fail("dsa: B and H must be <= 65535");
  // 1-D grids of (tile, head, batch) workgroups
  if ((int64_t)a->B * a->H * (((a->Lq > a->Lk ? a->Lq : a->Lk) + 127) / 128) > 0x7fffffff)
    return fail("dsa: B * H * tiles exceeds the 1-D grid range");
  if (!a->q || !a->k || !a->v || !a->out || !a->lse) return fail("dsa: q, k, v, out and lse are required");
  if ((a->flags & ~(DSA_C2P | DSA_P2C)) != 0) return fail("dsa: unknown flags 0x%x", a->flags);
  if (a->flags) {
    if (a->att_span < 1 || a->att_span > 16383) return fail("dsa: att_span must be in [1, 16383], got %d", a->att_span);
    if (!a->rel_table) return fail("dsa: rel_table is required when c2p/p2c is enabled");
  }
  if (a->dropout_threshold > 65535u)
    return fail("dsa: dropout_threshold must be in [0, 65535] (units of 1/65536), got %u", a->dropout_threshold);
  if (a->dtype == DSA_BF16 && a->out_lo && !aligned16(a->out_lo)) return fail("dsa: out_lo must be 16-byte aligned");
  if (a->dropout_threshold && a->dropout_bits && !aligned16(a->dropout_bits))
    return fail("dsa: dropout_bits must be 16-byte aligned");
  if ((a->flags & DSA_C2P) && !a->kr) return fail("dsa: c2p needs the pos-key table kr");
  // the forward addresses table rows with 32-bit element offsets
  if ((a->flags & DSA_C2P) && (int64_t)(2 * a->att_span - 1) * llabs(a->kr_strides[1]) + a->D > 0x7fffffffLL)
    return fail("dsa: kr row stride too large (rows of one head over 2^31 elements)");
  if ((a->flags & DSA_P2C) && (int64_t)(2 * a->att_span - 1) * llabs(a->qr_strides[1]) + a->D > 0x7fffffffLL)
    return fail("dsa: qr row stride too large (rows of one head over 2^31 elements)");
  if ((a->flags & DSA_P2C) && !a->qr) return fail("dsa: p2c needs the pos-query table qr");
  if ((a->key_keep ? 1 : 0) + (a->pair_keep ? 1 : 0) + (a->seg ? 1 : 0) > 1)
    return fail("dsa: give at most one of key_keep, pair_keep and seg");
  if ((a->key_keep || a->pair_keep || a->seg) && a->Lq != a->Lk)
    return fail("dsa: masks need Lq == Lk (query liveness is read from the key mask)");
  if (a->pair_keep) {  // the kernels read 16-byte chunks of the mask rows
    const int64_t k16 = (a->Lk + 15) / 16 * 16;
    if (!aligned16(a->pair_keep) || a->pair_keep_strides[0] % 16 || a->pair_keep_strides[1] % 16 ||
        a->pair_keep_stride_h % 16 ||
        (a->pair_keep_strides[1] != 0 ? a->pair_keep_strides[1] < k16 : a->Lk % 16 != 0))
      return fail("dsa: pair_keep must be 16-byte aligned, with batch, head and row strides multiples of 16 bytes "
                  "and each row's allocation reaching a multiple of 16 bytes past Lk");
  }
  if ((a->key_keep || a->seg) && a->Lk > 32768)  // per-tile lists in LDS
    return fail("dsa: key-padding and segment masks support sequences of at most 32768 tokens, got %d", a->Lk);
  const int vec = 16 / elem_bytes(a->dtype);
  const void* ptrs[] = {a->q, a->k, a->v, a->out};
  const int64_t* strides[] = {a->q_strides, a->k_strides, a->v_strides, a->o_strides};
  for (int t = 0; t < 4; ++t) {
    if (!aligned16(ptrs[t])) return fail("dsa: q/k/v/out must be 16-byte aligned");
    for (int s = 0; s < 3; ++s)
      if (strides[t][s] % vec != 0) return fail("dsa: q/k/v/out strides must be multiples of %d elements", vec);
  }
  if ((a->flags & DSA_C2P) && (!aligned16(a->kr) || a->kr_strides[0] % vec || a->kr_strides[1] % vec))
    return fail("dsa: kr must be 16-byte aligned with strides that are multiples of %d", vec);
  if ((a->flags & DSA_P2C) && (!aligned16(a->qr) || a->qr_strides[0] % vec || a->qr_strides[1] % vec))
    return fail("dsa: qr must be 16-byte aligned with strides that are multiples of %d", vec);
  return check_qc(a);
}

dsa::FwdParams to_params(const dsa_fwd_args* a) {
  dsa::FwdParams p;
  p.q = a->q;
  p.k = a->k;
  p.v = a->v;
  p.kr = a->kr;
  p.qr = a->qr;
  p.rel = a->rel_table;
  p.kk = a->key_keep;
  p.pk = a->pair_keep;
  p.out = a->out;
  p.lse = a->lse;
  p.bias = a->bias;
  for (int s = 0; s < 3; ++s) {
    p.qs[s] = a->q_strides[s];
    p.ks[s] = a->k_strides[s];
    p.vs[s] = a->v_strides[s];
    p.os[s] = a->o_strides[s];
  }
  for (int s = 0; s < 2; ++s) {
    p.krs[s] = a->kr_strides[s];
    p.qrs[s] = a->qr_strides[s];
  }
  p.krk = p.qrk = 64 / elem_bytes(a->dtype);  // rows contiguous: k-steps adjacent
  p.kkb = a->key_keep_stride_b;
  p.pkb = a->pair_keep_strides[0];
  p.pkq = a->pair_keep_strides[1];
  p.pkh = a->pair_keep ? a->pair_keep_stride_h : 0;
  p.seg = a->seg;
  p.segb = a->seg_stride_b;
  p.order = nullptr;
  p.qc = a->qc;
  for (int s = 0; s < 3; ++s) p.qcs[s] = a->qc ? a->qc_strides[s] : 0;
  p.B = a->B;
  p.H = a->H;
  p.Lq = a->Lq;
  p.Lk = a->Lk;
  p.A = a->flags ? a->att_span : 1;
  p.flags = a->flags;
  p.LqP = round_up(a->Lq, 128);
  p.LkP = round_up(a->Lk, 128);
  p.scale = a->scale;
  p.drop = nullptr;  // set where the keep bits are generated
  p.drop_scale = 1.f;
  p.olo = a->dtype == DSA_BF16 ? a->out_lo : nullptr;
  return p;
}

int mask_mode(const dsa_fwd_args* a) {
  return a->pair_keep ? dsa::MASK_PAIR : a->key_keep ? dsa::MASK_KEY : a->seg ? dsa::MASK_SEG : dsa::MASK_NONE;
}

int launch_check(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail("dsa: %s launch failed: %s", what, hipGetErrorString(e));
  return 0;
}

// Heaviest-first order (dsa_order.h) of B * ntiles items: cost and order
// arrays of that many ints each.  Used under key_keep / seg masks only, and
// for at most this many items (one block sorts them).
constexpr int64_t kMaxOrderItems = 65536;

size_t order_bytes(const dsa_fwd_args* a, int ntiles) {
  const int64_t n = (int64_t)a->B * ntiles;
  if (!(a->key_keep || a->seg) || n > kMaxOrderItems) return 0;
  return align_up((size_t)2 * n * sizeof(int), 256);
}

// Up to two heaviest-first orders (dsa_order.h): each job a buffer of cost
// then order (B * ntiles ints each), its tiles per row and its cost kind.
// fill_orders sets up the launches' parameters and the number of cost
// blocks (batch row fastest, then the tile group, then the job);
// launch_orders runs the cost and sort kernels, a caller that runs the cost
// blocks inside another launch only the sort (launch_order_sort).
int fill_orders(const dsa::FwdParams& p, int njobs, int* const* bufs, const int* ntiles, const bool* fwd,
                dsa::OrderParams2& op, int& ny) {
  op.f = p;
  op.njobs = njobs;
  int maxt = 0;
  for (int j = 0; j < 2; ++j) {
    const int jj = j < njobs ? j : 0;
    op.job[j].cost = bufs[jj];
    op.job[j].order = bufs[jj] + (int64_t)p.B * ntiles[jj];
    op.job[j].ntiles = ntiles[jj];
    op.job[j].fwd = fwd[jj] ? 1 : 0;
    maxt = std::max(maxt, ntiles[jj]);
  }
  ny = (maxt + dsa::ORDER_TPB - 1) / dsa::ORDER_TPB;
  return p.B * ny * njobs;
}

int launch_order_sort(const dsa::OrderParams2& op, hipStream_t st) {
  hipLaunchKernelGGL(dsa::dsa_order_sort_kernel, dim3(1), dim3(1024), 0, st, op);
  return launch_check("dsa_order_sort_kernel");
}

int launch_orders(const dsa::FwdParams& p, int njobs, int* const* bufs, const int* ntiles, const bool* fwd,
                  hipStream_t st) {
  dsa::OrderParams2 op;
  int ny = 0;
  fill_orders(p, njobs, bufs, ntiles, fwd, op, ny);
  const dim3 grid((unsigned)p.B, (unsigned)ny, (unsigned)njobs);
  hipLaunchKernelGGL(dsa::dsa_order_cost_kernel, grid, dim3(256), 0, st, op);
  if (launch_check("dsa_order_cost_kernel")) return 1;
  return launch_order_sort(op, st);
}

int fwd_tiles(const dsa_fwd_args* a) { return (a->Lq + dsa::dcfg::BQ - 1) / dsa::dcfg::BQ; }

// ---- attention dropout (dsa_dropout.h) ----
// Bytes of the keep bits (0 without dropout).
size_t drop_bits_bytes(const dsa_fwd_args* a) {
  if (!a->dropout_threshold) return 0;
  return dsa::dropout_bits_bytes(a->B, a->H, round_up(a->Lq, 128), round_up(a->Lk, 128));
}
// Bytes of them in the forward's or the backward's workspace: none when the
// caller keeps them (dropout_bits).
size_t drop_bytes(const dsa_fwd_args* a) {
  return a->dropout_bits ? 0 : align_up(drop_bits_bytes(a), 256);
}
float drop_scale(const dsa_fwd_args* a) { return 65536.f / (float)(65536u - a->dropout_threshold); }

// Generates the call's keep bits into `bits` and points the kernels'
// parameters at them.
int launch_dropout_bits(const dsa_fwd_args* a, uint32_t* bits, dsa::FwdParams& p, hipStream_t st) {
  dsa::DropParams d;
  d.bits = bits;
  d.B = a->B;
  d.H = a->H;
  d.NQB = round_up(a->Lq, 128) / 32;
  d.NKT = round_up(a->Lk, 128) / 64;
  d.t = a->dropout_threshold;
  d.k0 = (uint32_t)(a->dropout_seed & 0xffffffffu);
  d.k1 = (uint32_t)(a->dropout_seed >> 32);
  const dim3 grid((unsigned)((d.NKT + 3) / 4 * d.NQB), (unsigned)d.H, (unsigned)d.B);
  hipLaunchKernelGGL(dsa::dsa_dropout_bits_kernel, grid, dim3(256), 0, st, d);
  if (launch_check("dsa_dropout_bits_kernel")) return 1;
  p.drop = bits;
  p.drop_scale = drop_scale(a);
  return 0;
}


template <typename T, int D, int MASK, bool DROP>
int launch_fwd(const dsa::FwdParams& p, hipStream_t st) {
  dim3 grid((unsigned)((p.Lq + dsa::dcfg::BQ - 1) / dsa::dcfg::BQ * p.H * p.B));
  if (p.qc)
    hipLaunchKernelGGL((dsa::dsa_fwd_kernel<T, D, MASK, true, DROP>), grid, dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL((dsa::dsa_fwd_kernel<T, D, MASK, false, DROP>), grid, dim3(256), 0, st, p);
  return launch_check("dsa_fwd_kernel");
}

template <typename T, int D, int MASK>
int launch_fwd(const dsa::FwdParams& p, hipStream_t st) {
  return p.drop ? launch_fwd<T, D, MASK, true>(p, st) : launch_fwd<T, D, MASK, false>(p, st);
}

template <typename T, int D>
int fwd_mask(const dsa::FwdParams& p, int mode, hipStream_t st) {
  switch (mode) {
    case dsa::MASK_KEY: return launch_fwd<T, D, dsa::MASK_KEY>(p, st);
    case dsa::MASK_PAIR: return launch_fwd<T, D, dsa::MASK_PAIR>(p, st);
    case dsa::MASK_SEG: return launch_fwd<T, D, dsa::MASK_SEG>(p, st);
    default: return launch_fwd<T, D, dsa::MASK_NONE>(p, st);
  }
}

// Compute units of the current device (queried once per device).
int device_cus() {
  static std::atomic<int> cached[16] = {};
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (dev >= 0 && dev < 16 && (cus = cached[dev].load(std::memory_order_relaxed)) > 0) return cus;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) return 256;
  if (dev >= 0 && dev < 16) cached[dev].store(cus, std::memory_order_relaxed);
  return cus;
}

// Workspace of the backward (offsets 256-byte aligned) and the padded
// extents the kernels share.
struct WsLayout {
  int LqP, LkP, TGP, OFF, NDB, NPG;
  size_t rowinfo, krgt, qrgt, ds, gpart, seg, cinfo, korder, qorder, drop, total;
};

WsLayout ws_layout(const dsa_bwd_args* a) {
  const dsa_fwd_args& f = a->fwd;
  const size_t es = (size_t)elem_bytes(f.dtype);
  WsLayout w;
  w.LqP = round_up(f.Lq, 128);
  w.LkP = round_up(f.Lk, 128);
  w.OFF = w.LkP - 1;            // offset origin: t = d + OFF, 32-aligned tile starts
  w.TGP = w.LqP + w.LkP;        // offsets [-(LkP - 1), LqP] of every band window
  w.NDB = (w.LqP + w.LkP) / dsa::tbcfg::DBW;
  // Partial groups of the table kernel (ranges of an offset block's items
  // of one kind; a central block has about B * L / 32): about one and a
  // half workgroups per CU, whose fp32 atomics into the block accumulators
  // stay few and which leave room for dq beside them (B=32, L=512, the two
  // in one launch: backward 312 us with one workgroup per CU, 305 with one
  // and a half, 307 with two, 319 with three).  Long sequences and masks concentrate the work in the
  // central blocks, whose workgroups then bound the launch: those get at
  // most 64 items of a kind each.
  const int per = f.H * w.NDB;
  const int64_t items = (int64_t)f.B * ((w.LqP > w.LkP ? w.LqP : w.LkP) / 32);
  int64_t groups = (3 * device_cus() / 2 + per - 1) / per;
  if (w.NDB > 16 || f.key_keep || f.seg) groups = std::max<int64_t>(groups, (items + 63) / 64);
  w.NPG = (int)std::min<int64_t>(std::max<int64_t>(groups, 1), items);
  size_t off = 0;
  w.rowinfo = off;
  off = align_up(off + (size_t)f.B * f.H * w.LqP * 2 * sizeof(float), 256);
  w.krgt = off;
  if (f.flags & DSA_C2P) off = align_up(off + (size_t)f.H * f.D * w.TGP * es, 256);
  w.qrgt = off;
  if (f.flags & DSA_P2C) off = align_up(off + (size_t)f.H * f.D * w.TGP * es, 256);
  w.ds = off;
  off = align_up(off + (size_t)f.B * f.H * w.LkP * w.LqP * es, 256);
  w.gpart = off;
  if (f.flags) off = align_up(off + (size_t)f.H * w.NDB * 2 * dsa::tbcfg::DBW * f.D * sizeof(float), 256);
  w.seg = off;
  if (f.flags) off = align_up(off + (size_t)2 * 2 * (2 * f.att_span) * sizeof(int), 256);
  w.cinfo = off;
  if (f.key_keep || f.seg) off = align_up(off + (size_t)f.B * (w.LqP / 32) * 4 * sizeof(int), 256);
  w.korder = off;  // dkdv launch order (cost, order), under key_keep / seg
  off += order_bytes(&f, w.LkP / dsa::kvcfg::BKW);
  w.qorder = off;  // dq launch order
  off += order_bytes(&f, w.LqP / dsa::dqcfg::BQ);
  w.drop = off;  // attention dropout's keep bits, regenerated by PREP
  off += drop_bytes(&f);
  w.total = off;
  return w;
}

template <typename T, int D, bool DROP>
int launch_dkdv(const dsa::BwdParams& bp, const WsLayout& ws, int mode, hipStream_t st) {
  const dsa::FwdParams& f = bp.f;
  dim3 grid((unsigned)(ws.LkP / dsa::kvcfg::BKW * f.H * f.B));
  switch (mode) {
    case dsa::MASK_KEY:
      hipLaunchKernelGGL((dsa::dsa_bwd_dkdv_kernel<T, D, dsa::MASK_KEY, DROP>), grid, dim3(256), 0, st, bp);
      break;
    case dsa::MASK_PAIR:
      hipLaunchKernelGGL((dsa::dsa_bwd_dkdv_kernel<T, D, dsa::MASK_PAIR, DROP>), grid, dim3(256), 0, st, bp);
      break;
    case dsa::MASK_SEG:
      hipLaunchKernelGGL((dsa::dsa_bwd_dkdv_kernel<T, D, dsa::MASK_SEG, DROP>), grid, dim3(256), 0, st, bp);
      break;
    default:
      hipLaunchKernelGGL((dsa::dsa_bwd_dkdv_kernel<T, D, dsa::MASK_NONE, DROP>), grid, dim3(256), 0, st, bp);
  }
  return launch_check("dsa_bwd_dkdv_kernel");
}

template <typename T, int D>
int launch_bwd(const dsa_bwd_args* a, const WsLayout& ws, int mode, hipStream_t st) {
  const dsa_fwd_args& f = a->fwd;
  dsa::BwdParams bp;
  bp.f = to_params(&f);
  bp.dout = a->dout;
  for (int s = 0; s < 3; ++s) {
    bp.dos[s] = a->do_strides[s];
    bp.dqs[s] = a->dq_strides[s];
    bp.dks[s] = a->dk_strides[s];
    bp.dvs[s] = a->dv_strides[s];
  }
  bp.dq = a->dq;
  bp.dk = a->dk;
  bp.dv = a->dv;
  bp.dqc = f.qc ? a->dqc : nullptr;
  for (int s = 0; s < 3; ++s) bp.dqcs[s] = f.qc ? a->dqc_strides[s] : 0;
  bp.dkr = a->dkr;
  bp.dqr = a->dqr;
  bp.dtab_bf16 = a->dtab_dtype == DSA_BF16;
  bp.dtab_overwrite = a->dtab_overwrite != 0;
  char* base = static_cast<char*>(a->workspace);
  bp.rowinfo = reinterpret_cast<float*>(base + ws.rowinfo);
  bp.krgt = base + ws.krgt;
  bp.qrgt = base + ws.qrgt;
  bp.ds = base + ws.ds;
  bp.gpart = reinterpret_cast<float*>(base + ws.gpart);
  bp.rowseg = reinterpret_cast<int*>(base + ws.seg);
  bp.cinfo = (f.key_keep || f.seg) ? reinterpret_cast<int4*>(base + ws.cinfo) : nullptr;
  const int nkt = ws.LkP / dsa::kvcfg::BKW;
  int* kbuf = order_bytes(&f, nkt) ? reinterpret_cast<int*>(base + ws.korder) : nullptr;
  bp.korder = kbuf ? kbuf + (int64_t)f.B * nkt : nullptr;
  const int nqt = ws.LqP / dsa::dqcfg::BQ;
  int* qbuf = order_bytes(&f, nqt) ? reinterpret_cast<int*>(base + ws.qorder) : nullptr;
  bp.qorder = qbuf ? qbuf + (int64_t)f.B * nqt : nullptr;
  bp.TGP = ws.TGP;
  bp.OFF = ws.OFF;
  bp.NDB = ws.NDB;
  bp.NPG = ws.NPG;
  const int stages =
      a->stages ? a->stages : (DSA_STAGE_PREP | DSA_STAGE_DQ | DSA_STAGE_DKDV | DSA_STAGE_FOLD);
  if (f.dropout_threshold) {
    if (f.dropout_bits) {
      // the forward's keep bits, kept by the caller
      bp.f.drop = static_cast<const uint32_t*>(f.dropout_bits);
      bp.f.drop_scale = drop_scale(&f);
    } else {
      // PREP regenerates them (same seed, same bits) into the workspace; a
      // DKDV run in a later call reads the ones an earlier PREP left
      uint32_t* dbits = reinterpret_cast<uint32_t*>(base + ws.drop);
      if (stages & DSA_STAGE_PREP) {
        if (launch_dropout_bits(&f, dbits, bp.f, st)) return 1;
      } else {
        bp.f.drop = dbits;
        bp.f.drop_scale = drop_scale(&f);
      }
    }
  }

  if (stages & DSA_STAGE_PREP) {
    // dkdv's key tiles against 32-query chunks; dq's tiles (128 queries
    // against 64-key tiles) weigh as the forward's.  Their cost blocks run
    // first in the prep launch, the sort after it.
    int* bufs[2];
    int nts[2];
    bool kinds[2];
    int nj = 0;
    if (kbuf) bufs[nj] = kbuf, nts[nj] = nkt, kinds[nj++] = false;
    if (qbuf) bufs[nj] = qbuf, nts[nj] = nqt, kinds[nj++] = true;
    dsa::OrderParams2 op;
    op.f = bp.f;
    op.njobs = 0;
    dsa::PrepBlocks nb;
    nb.order = 0;
    nb.order_ny = 1;
    if (nj) nb.order = fill_orders(bp.f, nj, bufs, nts, kinds, op, nb.order_ny);
    const int64_t n = (int64_t)f.B * f.H * ws.LqP * (D / (16 / (int)sizeof(T)));
    nb.delta = (int)((n + 255) / 256);
    nb.gather = nb.seg = nb.chunk = nb.zero = 0;
    nb.gacc_floats = 0;
    if (f.key_keep || f.seg) nb.chunk = (int)(((int64_t)f.B * (ws.LqP / 32) + 255) / 256);
    if (f.flags) {
      const int64_t m = 2 * (int64_t)f.H * D * (ws.TGP / (16 / (int)sizeof(T)));
      nb.gather = (int)((m + 255) / 256);
      const int64_t ns = 2 * (int64_t)(f.Lq + f.Lk);
      nb.seg = (int)((ns + 255) / 256);
      // the table kernel's block accumulators, added to in FOLD
      nb.gacc_floats = (int64_t)f.H * ws.NDB * 2 * dsa::tbcfg::DBW * D;
      nb.zero = (int)((nb.gacc_floats / 4 + 255) / 256);
    }
    hipLaunchKernelGGL((dsa::dsa_bwd_prep_kernel<T, D>),
                       dim3((unsigned)(nb.order + nb.gather + nb.seg + nb.chunk + nb.zero + nb.delta)), dim3(256), 0, st,
                       bp, nb, op);
    if (launch_check("dsa_bwd_prep_kernel")) return 1;
    if (nj && launch_order_sort(op, st)) return 1;
  }
  if (stages & DSA_STAGE_DKDV) {
    if (bp.f.drop ? launch_dkdv<T, D, true>(bp, ws, mode, st) : launch_dkdv<T, D, false>(bp, ws, mode, st)) return 1;
  }
  // DQ and FOLD both only read dS: with both requested, the dq and table
  // workgroups run in one launch (dsa_bwd_dqtab.h) and share the GPU.
  // FOLD is TABLE (the table kernel) followed by SUM (the fold kernel).
  const bool fold = (stages & (DSA_STAGE_FOLD | DSA_STAGE_TABLE)) && f.flags;
  const bool sum = (stages & (DSA_STAGE_FOLD | DSA_STAGE_SUM)) && f.flags;
  const bool dq = (stages & DSA_STAGE_DQ) != 0;
  // dKr sums dS_ij times the c2p term's query rows: qc when it is given
  dsa::BwdParams tp = bp;
  if (f.qc) {
    tp.f.q = f.qc;
    for (int s = 0; s < 3; ++s) tp.f.qs[s] = f.qc_strides[s];
  }
  const int ntab = ws.NDB * f.H * ws.NPG;
  const int ndq = ws.LqP / dsa::dqcfg::BQ * f.H * f.B;
  if (fold && dq) {
    const int nt8 = (ntab + 7) / 8 * 8;
    const dim3 grid((unsigned)(nt8 + ndq));
    const bool listed = bp.cinfo != nullptr;
    if (listed && f.qc)
      hipLaunchKernelGGL((dsa::dsa_bwd_dqtab_kernel<T, D, true, true>), grid, dim3(256), 0, st, bp, tp, ntab, nt8, ndq);
    else if (listed)
      hipLaunchKernelGGL((dsa::dsa_bwd_dqtab_kernel<T, D, true, false>), grid, dim3(256), 0, st, bp, tp, ntab, nt8, ndq);
    else if (f.qc)
      hipLaunchKernelGGL((dsa::dsa_bwd_dqtab_kernel<T, D, false, true>), grid, dim3(256), 0, st, bp, tp, ntab, nt8, ndq);
    else
      hipLaunchKernelGGL((dsa::dsa_bwd_dqtab_kernel<T, D, false, false>), grid, dim3(256), 0, st, bp, tp, ntab, nt8, ndq);
    if (launch_check("dsa_bwd_dqtab_kernel")) return 1;
  } else if (fold) {
    if (bp.cinfo)
      hipLaunchKernelGGL((dsa::dsa_bwd_table_kernel<T, D, true>), dim3(ntab), dim3(256), 0, st, tp);
    else
      hipLaunchKernelGGL((dsa::dsa_bwd_table_kernel<T, D, false>), dim3(ntab), dim3(256), 0, st, tp);
    if (launch_check("dsa_bwd_table_kernel")) return 1;
  } else if (dq) {
    if (f.qc)
      hipLaunchKernelGGL((dsa::dsa_bwd_dq_kernel<T, D, true>), dim3(ndq), dim3(256), 0, st, bp);
    else
      hipLaunchKernelGGL((dsa::dsa_bwd_dq_kernel<T, D, false>), dim3(ndq), dim3(256), 0, st, bp);
    if (launch_check("dsa_bwd_dq_kernel")) return 1;
  }
  if (sum) {
    const int rows = 2 * f.H * (2 * f.att_span);
    if (f.Lq + f.Lk > 2048)  // long rows of saturated relative positions: four waves a row
      hipLaunchKernelGGL((dsa::dsa_bwd_fold_kernel<D, 4>), dim3((unsigned)rows), dim3(256), 0, st, bp);
    else  // one wave a row, four rows a workgroup
      hipLaunchKernelGGL((dsa::dsa_bwd_fold_kernel<D, 1>), dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st, bp);
    if (launch_check("dsa_bwd_fold_kernel")) return 1;
  }
  return 0;
}

static_assert(kStaticScratchBytes == 2 * kMaxOrderItems * sizeof(int), "the static scratch holds one launch order");

constexpr int kMaxDevices = 64;

// Per-device state of dsa_fwd_static: this GPU's address of `scratch` and an
// event recorded after each static forward (the next one, on any stream,
// waits for it: the calls share the array).  Set up once per device with
// that device current; a failed lookup is not kept, so a later call tries
// again.
struct StaticState {
  std::mutex mu;
  void* addr = nullptr;
  hipEvent_t done = nullptr;
};

StaticState& static_state(int dev) {
  static StaticState st[kMaxDevices];
  return st[dev];
}

// With the device's lock held: the scratch address (nullptr on failure).
void* static_scratch_locked(StaticState& s) {
  if (!s.addr) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) {
      (void)hipGetLastError();
      return nullptr;
    }
    s.addr = ptr;
  }
  if (!s.done && hipEventCreateWithFlags(&s.done, hipEventDisableTiming) != hipSuccess) {
    (void)hipGetLastError();
    s.done = nullptr;
  }
  return s.done ? s.addr : nullptr;
}

// Refuses a stream that is being captured into a HIP graph: capturing the
// library's launches ended in a host fault inside the runtime's capture end
// whose cause is not known, so the library does not run under capture.
int refuse_capture(hipStream_t st, const char* what) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  if (cs != hipStreamCaptureStatusNone)
    return fail("%s: the stream is capturing a HIP graph; the library's launches are not supported under graph capture",
                what);
  return 0;
}

// Bytes of the forward's k-step copy of one relative table (TableKs).
size_t table_ks_bytes(const dsa_fwd_args* a) {
  return align_up((size_t)a->H * (2 * a->att_span) * a->D * elem_bytes(a->dtype), 256);
}
size_t tables_ks_bytes(const dsa_fwd_args* a) {
  if (!a->flags) return 0;
  return table_ks_bytes(a) * (((a->flags & DSA_C2P) ? 1 : 0) + ((a->flags & DSA_P2C) ? 1 : 0));
}

// The forward with the launch-order scratch `order_buf` (NULL: no
// heaviest-first order), the scratch for the k-step copies of the relative
// tables `tab_buf` (NULL: the bands read the caller's tables) and, with
// dropout, the scratch for its keep bits `drop_buf`.  Arguments already
// checked.
int run_fwd(const dsa_fwd_args* a, int* order_buf, void* tab_buf, uint32_t* drop_buf, hipStream_t st) {
  dsa::FwdParams p = to_params(a);
  const int mode = mask_mode(a);
  if (drop_buf && launch_dropout_bits(a, drop_buf, p, st)) return 1;
  if (tab_buf && a->flags) {
    dsa::TableKs t;
    const int R = 2 * a->att_span, ks = 64 / elem_bytes(a->dtype);
    char* dst = static_cast<char*>(tab_buf);
    const bool has[2] = {(a->flags & DSA_C2P) != 0, (a->flags & DSA_P2C) != 0};
    const void* src[2] = {a->kr, a->qr};
    const int64_t* str[2] = {a->kr_strides, a->qr_strides};
    for (int k = 0; k < 2; ++k) {
      t.src[k] = has[k] ? src[k] : nullptr;
      t.hs[k] = str[k][0];
      t.rs[k] = str[k][1];
      t.dst[k] = has[k] ? dst : nullptr;
      if (has[k]) dst += table_ks_bytes(a);
    }
    t.H = a->H, t.R = R, t.D = a->D, t.esize = elem_bytes(a->dtype);
    const int64_t n = (int64_t)a->H * R * a->D * t.esize / 16;
    const int ncopy = (int)((n + 255) / 256);
    if (order_buf) {
      // the order's cost blocks in the same launch as the copies; the sort after it
      int* bufs[1] = {order_buf};
      const int nts[1] = {fwd_tiles(a)};
      const bool kinds[1] = {true};
      dsa::OrderParams2 op;
      int ny = 0;
      const int ncost = fill_orders(p, 1, bufs, nts, kinds, op, ny);
      hipLaunchKernelGGL(dsa::dsa_fwd_pre_kernel, dim3((unsigned)(ncost + 2 * ncopy)), dim3(256), 0, st, t, op, ncost,
                         ncopy);
      if (launch_check("dsa_fwd_pre_kernel")) return 1;
      if (launch_order_sort(op, st)) return 1;
      p.order = order_buf + (int64_t)a->B * fwd_tiles(a);
      order_buf = nullptr;  // done
    } else {
      hipLaunchKernelGGL(dsa::dsa_table_ks_kernel, dim3((unsigned)ncopy, 2), dim3(256), 0, st, t);
      if (launch_check("dsa_table_ks_kernel")) return 1;
    }
    // the bands read the copies: head stride NS * R * KS, row stride KS,
    // k-step stride R * KS
    const int64_t hs = (int64_t)(a->D / ks) * R * ks;
    if (has[0]) p.kr = t.dst[0], p.krs[0] = hs, p.krs[1] = ks, p.krk = (int64_t)R * ks;
    if (has[1]) p.qr = t.dst[1], p.qrs[0] = hs, p.qrs[1] = ks, p.qrk = (int64_t)R * ks;
  }
  if (order_buf) {
    int* bufs[1] = {order_buf};
    const int nts[1] = {fwd_tiles(a)};
    const bool kinds[1] = {true};
    if (launch_orders(p, 1, bufs, nts, kinds, st)) return 1;
    p.order = order_buf + (int64_t)a->B * fwd_tiles(a);
  }
  if (a->dtype == DSA_BF16) {
    return a->D == 64 ? fwd_mask<dsa::bf16, 64>(p, mode, st) : fwd_mask<dsa::bf16, 32>(p, mode, st);
  }
  return a->D == 64 ? fwd_mask<float, 64>(p, mode, st) : fwd_mask<float, 32>(p, mode, st);
}

// ---- fused row kernels (include/dsa_block.h) ------------------------------------------------
bool dtype_ok(int dt) { return dt == DSA_F32 || dt == DSA_BF16; }

// a tensor read or written in 4-element vectors along rows: base aligned to
// four elements, row stride a multiple of four
bool rows_ok(const void* p, int64_t stride, int dt) {
  const uintptr_t a = 4u * (uintptr_t)elem_bytes(dt);
  return p && (reinterpret_cast<uintptr_t>(p) % a) == 0 && stride % 4 == 0;
}
bool vec_ok(const void* p, int dt) { return !p || (reinterpret_cast<uintptr_t>(p) % (4u * (uintptr_t)elem_bytes(dt))) == 0; }

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

int reduce_cols(const float* part, int64_t nparts, int64_t stride, int K, int nout, const int64_t* off, void* const* out,
                int dt, hipStream_t st) {
  dsa::rows::ReduceCols rc;
  rc.part = part;
  rc.nparts = nparts;
  rc.stride = stride;
  rc.K = K;
  rc.nout = nout;
  for (int j = 0; j < 3; ++j) {
    rc.off[j] = j < nout ? off[j] : 0;
    rc.out[j] = j < nout ? out[j] : nullptr;
  }
  rc.dt = dt;
  hipLaunchKernelGGL(dsa::rows::reduce_cols_kernel, dim3((unsigned)cdiv(K, 64), (unsigned)nout), dim3(64 * dsa::rows::RED_W), 0,
                     st, rc);
  return launch_check("reduce_cols_kernel");
}

int check_ln(const dsa_ln_args* a, bool bwd) {
  if (!a) return fail("dsa: null arguments");
  if (a->N < 1 || a->C < 4 || a->C % 4 || a->C > 2048)
    return fail("dsa_add_ln: N >= 1 and C a multiple of 4 in [4, 2048] required, got N=%lld C=%d", (long long)a->N, a->C);
  if (!dtype_ok(a->x_dtype) || !dtype_ok(a->param_dtype) || (a->res && !dtype_ok(a->res_dtype)))
    return fail("dsa_add_ln: unsupported dtype");
  if (!rows_ok(a->x, a->x_stride, a->x_dtype)) return fail("dsa_add_ln: x must be aligned to 4 elements with a row stride a multiple of 4");
  if (!a->gamma || !a->beta || !vec_ok(a->gamma, a->param_dtype) || !vec_ok(a->beta, a->param_dtype) || !vec_ok(a->bias, a->param_dtype))
    return fail("dsa_add_ln: gamma and beta (and bias) must be given and aligned to 4 elements");
  if (a->res && (a->rows_per_group < 1 || !vec_ok(a->res, a->res_dtype) || a->res_strides[0] % 4 || a->res_strides[1] % 4))
    return fail("dsa_add_ln: res needs rows_per_group >= 1, 4-element alignment and strides multiples of 4");
  if (!a->mean || !a->rstd) return fail("dsa_add_ln: mean and rstd are required");
  if (!bwd) {
    if (!dtype_ok(a->y_dtype) || !rows_ok(a->y, a->y_stride, a->y_dtype)) return fail("dsa_add_ln: bad y");
    return 0;
  }
  if (!dtype_ok(a->dy_dtype) || !rows_ok(a->dy, a->dy_stride, a->dy_dtype)) return fail("dsa_add_ln: bad dy");
  if (a->dz_dtype != a->x_dtype || !rows_ok(a->dz, a->dz_stride, a->dz_dtype)) return fail("dsa_add_ln: bad dz (x's dtype)");
  const size_t need = dsa_block_workspace_bytes(DSA_BLOCK_LN, a->N, a->C);
  if (!a->workspace || a->workspace_bytes < need || !aligned16(a->workspace))
    return fail("dsa_add_ln: workspace of %zu bytes (16-byte aligned) required", need);
  return 0;
}

dsa::rows::LnParams ln_params(const dsa_ln_args* a) {
  dsa::rows::LnParams p;
  p.x = a->x;
  p.bias = a->bias;
  p.res = a->res;
  p.gamma = a->gamma;
  p.beta = a->beta;
  p.dy = a->dy;
  p.y = a->y;
  p.dz = a->dz;
  p.dgamma = a->dgamma;
  p.dbeta = a->dbeta;
  p.dbias = a->dbias;
  p.mean = a->mean;
  p.rstd = a->rstd;
  p.part = static_cast<float*>(a->workspace);
  p.xs = a->x_stride;
  p.rs0 = a->res_strides[0];
  p.rs1 = a->res_strides[1];
  p.rpg = a->res ? a->rows_per_group : 1;
  p.ys = a->y_stride;
  p.dys = a->dy_stride;
  p.dzs = a->dz_stride;
  p.N = a->N;
  p.C = a->C;
  p.pdt = a->param_dtype;
  p.eps = a->eps;
  return p;
}

int check_gelu(const dsa_gelu_args* a, bool bwd) {
  if (!a) return fail("dsa: null arguments");
  if (a->N < 1 || a->C < 4 || a->C % 4) return fail("dsa_bias_gelu: N >= 1 and C a multiple of 4 required");
  if (!dtype_ok(a->x_dtype) || !dtype_ok(a->param_dtype)) return fail("dsa_bias_gelu: unsupported dtype");
  if (!rows_ok(a->x, a->x_stride, a->x_dtype) || !vec_ok(a->bias, a->param_dtype)) return fail("dsa_bias_gelu: bad x or bias");
  if (!bwd) return (!dtype_ok(a->y_dtype) || !rows_ok(a->y, a->y_stride, a->y_dtype)) ? fail("dsa_bias_gelu: bad y") : 0;
  if (!dtype_ok(a->dy_dtype) || !rows_ok(a->dy, a->dy_stride, a->dy_dtype)) return fail("dsa_bias_gelu: bad dy");
  if (a->dz_dtype != a->x_dtype || !rows_ok(a->dz, a->dz_stride, a->dz_dtype)) return fail("dsa_bias_gelu: bad dz (x's dtype)");
  const size_t need = dsa_block_workspace_bytes(DSA_BLOCK_GELU, a->N, a->C);
  if (!a->workspace || a->workspace_bytes < need || !aligned16(a->workspace))
    return fail("dsa_bias_gelu: workspace of %zu bytes (16-byte aligned) required", need);
  return 0;
}

// The 8-wide GELU kernels: rows in 8-element vectors (C, the row strides and
// the tensors' element offsets multiples of 8; the bias, in its own dtype,
// too).
bool gelu_wide(const dsa_gelu_args* a, bool bwd) {
  auto ok8 = [](const void* p, int64_t stride, int dt) {
    return !p || ((reinterpret_cast<uintptr_t>(p) % (8u * (uintptr_t)elem_bytes(dt))) == 0 && stride % 8 == 0);
  };
  if (a->C % 8 || !ok8(a->x, a->x_stride, a->x_dtype) || !ok8(a->bias, 0, a->param_dtype)) return false;
  if (!bwd) return ok8(a->y, a->y_stride, a->y_dtype);
  return ok8(a->dy, a->dy_stride, a->dy_dtype) && ok8(a->dz, a->dz_stride, a->dz_dtype);
}

dsa::rows::GeluParams gelu_params(const dsa_gelu_args* a) {
  dsa::rows::GeluParams p;
  p.x = a->x;
  p.bias = a->bias;
  p.dy = a->dy;
  p.y = a->y;
  p.dz = a->dz;
  p.dbias = a->dbias;
  p.part = static_cast<float*>(a->workspace);
  p.xs = a->x_stride;
  p.ys = a->y_stride;
  p.dys = a->dy_stride;
  p.dzs = a->dz_stride;
  p.N = a->N;
  p.C = a->C;
  p.pdt = a->param_dtype;
  return p;
}

int check_rtd(const dsa_rtd_args* a, bool bwd) {
  if (!a) return fail("dsa: null arguments");
  if (a->N < 1 || a->C < 4 || a->C % 4 || a->C > 2048)
    return fail("dsa_rtd_loss: N >= 1 and C a multiple of 4 in [4, 2048] required");
  if (!dtype_ok(a->x_dtype) || !dtype_ok(a->param_dtype)) return fail("dsa_rtd_loss: unsupported dtype");
  if (!rows_ok(a->x, a->x_stride, a->x_dtype) || !a->w || !vec_ok(a->w, a->param_dtype) || !a->labels)
    return fail("dsa_rtd_loss: x, w and labels are required (x and w aligned to 4 elements)");
  if (!a->logits || !a->denom) return fail("dsa_rtd_loss: logits and denom are required");
  const size_t need = dsa_block_workspace_bytes(DSA_BLOCK_RTD, a->N, a->C);
  if (!a->workspace || a->workspace_bytes < need || !aligned16(a->workspace))
    return fail("dsa_rtd_loss: workspace of %zu bytes (16-byte aligned) required", need);
  if (!bwd) return a->loss ? 0 : fail("dsa_rtd_loss: loss is required");
  if (!a->dloss || !a->dw) return fail("dsa_rtd_loss: dloss and dw are required");
  if (!dtype_ok(a->dx_dtype) || !rows_ok(a->dx, a->dx_stride, a->dx_dtype)) return fail("dsa_rtd_loss: bad dx");
  return 0;
}

dsa::rows::RtdParams rtd_params(const dsa_rtd_args* a) {
  dsa::rows::RtdParams p;
  p.x = a->x;
  p.w = a->w;
  p.b = a->b;
  p.labels = a->labels;
  p.active = a->active;
  p.logits = a->logits;
  p.loss = a->loss;
  p.denom = a->denom;
  p.part = static_cast<float*>(a->workspace);
  p.dloss = a->dloss;
  p.dx = a->dx;
  p.dw = a->dw;
  p.db = a->db;
  p.xs = a->x_stride;
  p.dxs = a->dx_stride;
  p.N = a->N;
  p.C = a->C;
  p.pdt = a->param_dtype;
  return p;
}

}  // namespace

extern "C" {

int dsa_version(void) { return 11; }

const char* dsa_last_error(void) { return g_err.c_str(); }

int dsa_fwd(const dsa_fwd_args* a, void* stream) {
  g_err.clear();
  if (check_fwd(a)) return 1;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (refuse_capture(st, "dsa_fwd")) return 1;
  const size_t ob = order_bytes(a, fwd_tiles(a)), tb = tables_ks_bytes(a), db = drop_bytes(a);
  if (db && (!a->workspace || a->workspace_bytes < ob + tb + db))
    return fail("dsa: attention dropout needs dropout_bits or the forward workspace of %zu bytes (its keep bits), "
                "got %zu", ob + tb + db, a->workspace ? a->workspace_bytes : (size_t)0);
  int* buf = nullptr;
  void* tabs = nullptr;
  uint32_t* dbits = nullptr;
  if (a->workspace && (ob || tb || db)) {
    if (a->workspace_bytes < ob) return fail("dsa: forward workspace of %zu bytes required, got %zu", ob, a->workspace_bytes);
    if (!aligned16(a->workspace)) return fail("dsa: forward workspace must be 16-byte aligned");
    if (ob) buf = static_cast<int*>(a->workspace);
    // a workspace of the size without the table copies (earlier versions of
    // dsa_fwd_workspace_bytes) runs the bands on the caller's tables
    if (tb && a->workspace_bytes >= ob + tb) tabs = static_cast<char*>(a->workspace) + ob;
    if (db) dbits = reinterpret_cast<uint32_t*>(static_cast<char*>(a->workspace) + ob + tb);
  }
  if (a->dropout_threshold && a->dropout_bits) dbits = static_cast<uint32_t*>(a->dropout_bits);
  return run_fwd(a, buf, tabs, dbits, st);
}

int dsa_fwd_static(const dsa_fwd_args* a, void* stream) {
  g_err.clear();
  if (check_fwd(a)) return 1;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (refuse_capture(st, "dsa_fwd_static")) return 1;
  if (a->dropout_threshold)
    return fail("dsa_fwd_static: attention dropout needs dsa_fwd and its workspace (the keep bits)");
  if (!(a->key_keep || a->seg)) return run_fwd(a, nullptr, nullptr, nullptr, st);  // no scratch used
  const int64_t n = (int64_t)a->B * fwd_tiles(a);
  if (n > kMaxOrderItems)
    return fail("dsa_fwd_static: B * ceil(Lq / 128) = %lld launch-order items exceed the static scratch's "
                "%lld (%zu bytes); use dsa_fwd with a caller workspace",
                (long long)n, (long long)kMaxOrderItems, kStaticScratchBytes);
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail("dsa_fwd_static: no current device below %d (got %d)", kMaxDevices, dev);
  StaticState& s = static_state(dev);
  // The lock orders the calls of this process on the device: each waits on
  // its stream for the previous static forward (on any stream) and records
  // its own end, so no two of them use the array at once.
  std::lock_guard<std::mutex> lock(s.mu);
  int* buf = static_cast<int*>(static_scratch_locked(s));
  if (!buf) return fail("dsa_fwd_static: no address for the static scratch (or its event) on device %d", dev);
  if (hipStreamWaitEvent(st, s.done, 0) != hipSuccess) return fail("dsa_fwd_static: hipStreamWaitEvent failed");
  const int rc = run_fwd(a, buf, nullptr, nullptr, st);
  if (hipEventRecord(s.done, st) != hipSuccess) {
    (void)hipGetLastError();
    return rc ? rc : fail("dsa_fwd_static: hipEventRecord failed");
  }
  return rc;
}

int dsa_bias(const dsa_fwd_args* a, void* out, const int64_t* out_strides, void* stream) {
  g_err.clear();
  if (!a) return fail("dsa: null arguments");
  if (a->dtype != DSA_BF16 && a->dtype != DSA_F32) return fail("dsa: unsupported dtype %d", a->dtype);
  if (a->D != 32 && a->D != 64) return fail("dsa: head dim must be 32 or 64, got %d", a->D);
  if (a->B < 1 || a->H < 1 || a->Lq < 1 || a->Lk < 1)
    return fail("dsa: empty shape B=%d H=%d Lq=%d Lk=%d", a->B, a->H, a->Lq, a->Lk);
  if (a->B > 65535 || a->H > 65535) return fail("dsa: B and H must be <= 65535");
  const int64_t nqt = (a->Lq + dsa::dcfg::BQ - 1) / dsa::dcfg::BQ, nkt = (a->Lk + dsa::dcfg::BK - 1) / dsa::dcfg::BK;
  if ((int64_t)a->B * a->H * nqt * nkt > 0x7fffffff) return fail("dsa: B * H * tiles exceeds the 1-D grid range");
  if (!a->q || !a->k || !out || !out_strides) return fail("dsa: q, k, out and out_strides are required");
  if ((a->flags & ~(DSA_C2P | DSA_P2C)) != 0) return fail("dsa: unknown flags 0x%x", a->flags);
  if (a->flags) {
    if (a->att_span < 1 || a->att_span > 16383) return fail("dsa: att_span must be in [1, 16383], got %d", a->att_span);
    if (!a->rel_table) return fail("dsa: rel_table is required when c2p/p2c is enabled");
  }
  if ((a->flags & DSA_C2P) && !a->kr) return fail("dsa: c2p needs the pos-key table kr");
  if ((a->flags & DSA_P2C) && !a->qr) return fail("dsa: p2c needs the pos-query table qr");
  if ((a->flags & DSA_C2P) && (int64_t)(2 * a->att_span - 1) * llabs(a->kr_strides[1]) + a->D > 0x7fffffffLL)
    return fail("dsa: kr row stride too large (rows of one head over 2^31 elements)");
  if ((a->flags & DSA_P2C) && (int64_t)(2 * a->att_span - 1) * llabs(a->qr_strides[1]) + a->D > 0x7fffffffLL)
    return fail("dsa: qr row stride too large (rows of one head over 2^31 elements)");
  const int vec = 16 / elem_bytes(a->dtype);
  if (!aligned16(a->q) || !aligned16(a->k)) return fail("dsa: q and k must be 16-byte aligned");
  for (int s = 0; s < 3; ++s)
    if (a->q_strides[s] % vec || a->k_strides[s] % vec)
      return fail("dsa: q / k strides must be multiples of %d elements", vec);
  if ((a->flags & DSA_C2P) && (!aligned16(a->kr) || a->kr_strides[0] % vec || a->kr_strides[1] % vec))
    return fail("dsa: kr must be 16-byte aligned with strides that are multiples of %d", vec);
  if ((a->flags & DSA_P2C) && (!aligned16(a->qr) || a->qr_strides[0] % vec || a->qr_strides[1] % vec))
    return fail("dsa: qr must be 16-byte aligned with strides that are multiples of %d", vec);
  if (check_qc(a)) return 1;
  if ((reinterpret_cast<uintptr_t>(out) % elem_bytes(a->dtype)) != 0) return fail("dsa: out must be aligned to its element size");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (refuse_capture(st, "dsa_bias")) return 1;
  dsa::BiasParams bp;
  bp.f = to_params(a);
  bp.out = out;
  for (int s = 0; s < 3; ++s) bp.obs[s] = out_strides[s];
  const dim3 grid((unsigned)(a->B * (int64_t)a->H * nqt * nkt));
  const bool qc = a->qc != nullptr;
  if (a->dtype == DSA_BF16) {
    if (a->D == 64) {
      if (qc) hipLaunchKernelGGL((dsa::dsa_bias_kernel<dsa::bf16, 64, true>), grid, dim3(256), 0, st, bp);
      else hipLaunchKernelGGL((dsa::dsa_bias_kernel<dsa::bf16, 64, false>), grid, dim3(256), 0, st, bp);
    } else {
      if (qc) hipLaunchKernelGGL((dsa::dsa_bias_kernel<dsa::bf16, 32, true>), grid, dim3(256), 0, st, bp);
      else hipLaunchKernelGGL((dsa::dsa_bias_kernel<dsa::bf16, 32, false>), grid, dim3(256), 0, st, bp);
    }
  } else {
    if (a->D == 64) {
      if (qc) hipLaunchKernelGGL((dsa::dsa_bias_kernel<float, 64, true>), grid, dim3(256), 0, st, bp);
      else hipLaunchKernelGGL((dsa::dsa_bias_kernel<float, 64, false>), grid, dim3(256), 0, st, bp);
    } else {
      if (qc) hipLaunchKernelGGL((dsa::dsa_bias_kernel<float, 32, true>), grid, dim3(256), 0, st, bp);
      else hipLaunchKernelGGL((dsa::dsa_bias_kernel<float, 32, false>), grid, dim3(256), 0, st, bp);
    }
  }
  return launch_check("dsa_bias_kernel");
}

size_t dsa_fwd_bias_bytes(const dsa_fwd_args* a) {
  if (!a || !a->flags) return 0;
  return (size_t)a->B * a->H * round_up(a->Lq, 128) * round_up(a->Lk, 128) * (a->dtype == DSA_BF16 ? 2 : 4);
}

size_t dsa_fwd_dropout_bytes(const dsa_fwd_args* a) {
  if (!a || a->B < 1 || a->Lq < 1 || a->Lk < 1 || a->H < 1) return 0;
  return drop_bits_bytes(a);
}

size_t dsa_fwd_workspace_bytes(const dsa_fwd_args* a) {
  if (!a || a->B < 1 || a->Lq < 1 || a->H < 1 || a->D < 1) return 0;
  if (a->flags && (a->att_span < 1 || a->att_span > 16383)) return 0;
  return order_bytes(a, fwd_tiles(a)) + tables_ks_bytes(a) + drop_bytes(a);
}

size_t dsa_bwd_workspace_bytes(const dsa_bwd_args* a) {
  if (!a) return 0;
  return ws_layout(a).total;
}

int dsa_bwd(const dsa_bwd_args* a, void* stream) {
  g_err.clear();
  if (!a) return fail("dsa: null arguments");
  constexpr int kStages = DSA_STAGE_PREP | DSA_STAGE_DQ | DSA_STAGE_DKDV | DSA_STAGE_FOLD | DSA_STAGE_TABLE | DSA_STAGE_SUM;
  if (a->stages & ~kStages) return fail("dsa: unknown backward stage bits 0x%x", (unsigned)(a->stages & ~kStages));
  if (check_fwd(&a->fwd)) return 1;
  const dsa_fwd_args& f = a->fwd;
  if (!a->dout || !a->dq || !a->dk || !a->dv) return fail("dsa: dout, dq, dk and dv are required");
  if ((f.flags & DSA_C2P) && !a->dkr) return fail("dsa: c2p backward needs dkr");
  if ((f.flags & DSA_P2C) && !a->dqr) return fail("dsa: p2c backward needs dqr");
  if (a->dtab_dtype != DSA_F32 && a->dtab_dtype != DSA_BF16) return fail("dsa: unsupported dtab_dtype %d", a->dtab_dtype);
  if (a->dtab_dtype == DSA_BF16 && !a->dtab_overwrite)
    return fail("dsa: bf16 table gradients are written, not accumulated (set dtab_overwrite)");
  if (f.flags && !f.bias) return fail("dsa: the backward needs the relative term saved by dsa_fwd (fwd.bias)");
  if (f.qc) {
    const int v = 16 / elem_bytes(f.dtype);
    if (!a->dqc || !aligned16(a->dqc)) return fail("dsa: with fwd.qc the backward needs dqc (16-byte aligned)");
    for (int s = 0; s < 3; ++s)
      if (a->dqc_strides[s] % v != 0) return fail("dsa: dqc strides must be multiples of %d elements", v);
  }
  if (f.flags && !aligned16(f.bias)) return fail("dsa: fwd.bias must be 16-byte aligned");
  const int vec = 16 / elem_bytes(f.dtype);
  const void* ptrs[] = {a->dout, a->dq, a->dk, a->dv};
  const int64_t* strides[] = {a->do_strides, a->dq_strides, a->dk_strides, a->dv_strides};
  for (int t = 0; t < 4; ++t) {
    if (!aligned16(ptrs[t])) return fail("dsa: dout/dq/dk/dv must be 16-byte aligned");
    for (int s = 0; s < 3; ++s)
      if (strides[t][s] % vec != 0) return fail("dsa: dout/dq/dk/dv strides must be multiples of %d elements", vec);
  }
  const WsLayout ws = ws_layout(a);
  // the table kernel addresses one (b, h) slice of dS, and the rows of q and
  // k of one (b, h), with 32-bit byte offsets
  const int64_t es = elem_bytes(f.dtype);
  if ((int64_t)ws.LqP * ws.LkP * es > 0x7fffffffLL)
    return fail("dsa: Lq x Lk too large for the backward (padded (b, h) slice of dS over 2 GiB)");
  if (((int64_t)(f.Lq - 1) * f.q_strides[1] + f.D) * es > 0x7fffffffLL ||
      ((int64_t)(f.Lk - 1) * f.k_strides[1] + f.D) * es > 0x7fffffffLL)
    return fail("dsa: q / k sequence stride too large for the backward (rows of one (b, h) over 2 GiB)");
  if (!a->workspace || a->workspace_bytes < ws.total)
    return fail("dsa: workspace of %zu bytes required, got %zu", ws.total, a->workspace_bytes);
  if (!aligned16(a->workspace)) return fail("dsa: workspace must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (refuse_capture(st, "dsa_bwd")) return 1;
  const int mode = mask_mode(&f);
  if (f.dtype == DSA_BF16) {
    return f.D == 64 ? launch_bwd<dsa::bf16, 64>(a, ws, mode, st) : launch_bwd<dsa::bf16, 32>(a, ws, mode, st);
  }
  return f.D == 64 ? launch_bwd<float, 64>(a, ws, mode, st) : launch_bwd<float, 32>(a, ws, mode, st);
}

}  // extern "C"

namespace {
// Calls f(std::integral_constant<int, NC>) for NC = ceil(C / 256), the
// 4-element chunks a lane holds in the row kernels (C <= 2048 is checked
// before).
template <typename F>
void by_chunks(int C, F f) {
  switch (cdiv(C, 256)) {
    case 1: f(std::integral_constant<int, 1>{}); break;
    case 2: f(std::integral_constant<int, 2>{}); break;
    case 3: f(std::integral_constant<int, 3>{}); break;
    case 4: f(std::integral_constant<int, 4>{}); break;
    case 5:
    case 6: f(std::integral_constant<int, 6>{}); break;
    default: f(std::integral_constant<int, 8>{}); break;
  }
}

template <typename T>
struct Tag {
  typedef T type;
};
// Calls f(Tag<element type>) for a row tensor's dtype (DSA_BF16 or DSA_F32).
template <typename F>
void by_dtype(int dt, F f) {
  if (dt == DSA_BF16) f(Tag<dsa::bf16>{});
  else f(Tag<float>{});
}
}  // namespace

extern "C" {

size_t dsa_block_workspace_bytes(int kind, int64_t N, int32_t C) {
  if (N < 1 || C < 1) return 0;
  switch (kind) {
    case DSA_BLOCK_LN: return align_up((size_t)cdiv(N, dsa::rows::LN_RB) * 3 * C * sizeof(float), 256);
    case DSA_BLOCK_GELU: return align_up((size_t)cdiv(N, dsa::rows::GELU_RB) * C * sizeof(float), 256);
    case DSA_BLOCK_RTD: {
      const int64_t nb = cdiv(N, dsa::rows::RTD_RB);
      return align_up((size_t)nb * (size_t)std::max<int64_t>(2, C + 1) * sizeof(float), 256);
    }
    default: return 0;
  }
}

int dsa_add_ln_fwd(const dsa_ln_args* a, void* stream) {
  g_err.clear();
  if (check_ln(a, false)) return 1;
  if (refuse_capture(static_cast<hipStream_t>(stream), "dsa_add_ln_fwd")) return 1;
  const dsa::rows::LnParams p = ln_params(a);
  by_chunks(a->C, [&](auto nc) {
    by_dtype(a->x_dtype, [&](auto tx) {
      by_dtype(a->res ? a->res_dtype : a->x_dtype, [&](auto tr) {
        by_dtype(a->y_dtype, [&](auto ty) {
          auto k = dsa::rows::ln_fwd_kernel<decltype(nc)::value, typename decltype(tx)::type, typename decltype(tr)::type,
                                            typename decltype(ty)::type>;
          hipLaunchKernelGGL(k, dim3((unsigned)cdiv(a->N, 4)), dim3(256), 0, static_cast<hipStream_t>(stream), p);
        });
      });
    });
  });
  return launch_check("ln_fwd_kernel");
}

int dsa_add_ln_bwd(const dsa_ln_args* a, void* stream) {
  g_err.clear();
  if (check_ln(a, true)) return 1;
  if (refuse_capture(static_cast<hipStream_t>(stream), "dsa_add_ln_bwd")) return 1;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dsa::rows::LnParams p = ln_params(a);
  const int64_t nb = cdiv(a->N, dsa::rows::LN_RB);
  by_chunks(a->C, [&](auto nc) {
    by_dtype(a->x_dtype, [&](auto tx) {
      by_dtype(a->res ? a->res_dtype : a->x_dtype, [&](auto tr) {
        by_dtype(a->dy_dtype, [&](auto tdy) {
          auto k = dsa::rows::ln_bwd_kernel<decltype(nc)::value, typename decltype(tx)::type, typename decltype(tr)::type,
                                            typename decltype(tdy)::type>;
          hipLaunchKernelGGL(k, dim3((unsigned)nb), dim3(256), 0, st, p);
        });
      });
    });
  });
  if (launch_check("ln_bwd_kernel")) return 1;
  const int64_t off[3] = {0, a->C, 2 * (int64_t)a->C};
  void* const out[3] = {a->dgamma, a->dbeta, a->dbias};
  return reduce_cols(p.part, nb, 3 * (int64_t)a->C, a->C, 3, off, out, a->param_dtype, st);
}

int dsa_bias_gelu_fwd(const dsa_gelu_args* a, void* stream) {
  g_err.clear();
  if (check_gelu(a, false)) return 1;
  if (refuse_capture(static_cast<hipStream_t>(stream), "dsa_bias_gelu_fwd")) return 1;
  const dsa::rows::GeluParams p = gelu_params(a);
  if (cdiv(a->N, dsa::rows::GELU_RB) > 65535)
    return fail("dsa_bias_gelu: N too large (%lld rows, at most %d)", (long long)a->N, 65535 * dsa::rows::GELU_RB);
  const bool wide = gelu_wide(a, false);
  by_dtype(a->x_dtype, [&](auto tx) {
    by_dtype(a->y_dtype, [&](auto ty) {
      typedef typename decltype(tx)::type TX;
      typedef typename decltype(ty)::type TY;
      const dim3 rows_grid((unsigned)cdiv(a->N, dsa::rows::GELU_RB));
      if (wide)
        hipLaunchKernelGGL((dsa::rows::gelu8_fwd_kernel<TX, TY>), dim3((unsigned)cdiv(a->C, 1024), rows_grid.x), dim3(128),
                           0, static_cast<hipStream_t>(stream), p);
      else
        hipLaunchKernelGGL((dsa::rows::gelu_fwd_kernel<TX, TY>), dim3((unsigned)cdiv(a->C / 4, 256), rows_grid.x),
                           dim3(256), 0, static_cast<hipStream_t>(stream), p);
    });
  });
  return launch_check("gelu_fwd_kernel");
}

int dsa_bias_gelu_bwd(const dsa_gelu_args* a, void* stream) {
  g_err.clear();
  if (check_gelu(a, true)) return 1;
  if (refuse_capture(static_cast<hipStream_t>(stream), "dsa_bias_gelu_bwd")) return 1;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dsa::rows::GeluParams p = gelu_params(a);
  const int64_t nb = cdiv(a->N, dsa::rows::GELU_RB);
  if (nb > 65535) return fail("dsa_bias_gelu: N too large (%lld rows, at most %d)", (long long)a->N, 65535 * dsa::rows::GELU_RB);
  const bool wide = gelu_wide(a, true);
  by_dtype(a->x_dtype, [&](auto tx) {
    by_dtype(a->dy_dtype, [&](auto tdy) {
      typedef typename decltype(tx)::type TX;
      typedef typename decltype(tdy)::type TDY;
      if (wide)
        hipLaunchKernelGGL((dsa::rows::gelu8_bwd_kernel<TX, TDY>), dim3((unsigned)cdiv(a->C, 1024), (unsigned)nb), dim3(128),
                           0, st, p);
      else
        hipLaunchKernelGGL((dsa::rows::gelu_bwd_kernel<TX, TDY>), dim3((unsigned)cdiv(a->C / 4, 256), (unsigned)nb),
                           dim3(256), 0, st, p);
    });
  });
  if (launch_check("gelu_bwd_kernel")) return 1;
  if (!a->dbias) return 0;
  const int64_t off[1] = {0};
  void* const out[1] = {a->dbias};
  return reduce_cols(p.part, nb, a->C, a->C, 1, off, out, a->param_dtype, st);
}

int dsa_rtd_loss_fwd(const dsa_rtd_args* a, void* stream) {
  g_err.clear();
  if (check_rtd(a, false)) return 1;
  if (refuse_capture(static_cast<hipStream_t>(stream), "dsa_rtd_loss_fwd")) return 1;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dsa::rows::RtdParams p = rtd_params(a);
  const int64_t nb = cdiv(a->N, dsa::rows::RTD_RB);
  by_chunks(a->C, [&](auto nc) {
    by_dtype(a->x_dtype, [&](auto tx) {
      auto k = dsa::rows::rtd_fwd_kernel<decltype(nc)::value, typename decltype(tx)::type>;
      hipLaunchKernelGGL(k, dim3((unsigned)nb), dim3(256), 0, st, p);
    });
  });
  if (launch_check("rtd_fwd_kernel")) return 1;
  hipLaunchKernelGGL(dsa::rows::rtd_loss_kernel, dim3(1), dim3(64), 0, st, p, (int)nb);
  return launch_check("rtd_loss_kernel");
}

int dsa_rtd_loss_bwd(const dsa_rtd_args* a, void* stream) {
  g_err.clear();
  if (check_rtd(a, true)) return 1;
  if (refuse_capture(static_cast<hipStream_t>(stream), "dsa_rtd_loss_bwd")) return 1;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dsa::rows::RtdParams p = rtd_params(a);
  const int64_t nb = cdiv(a->N, dsa::rows::RTD_RB);
  by_chunks(a->C, [&](auto nc) {
    by_dtype(a->x_dtype, [&](auto tx) {
      by_dtype(a->dx_dtype, [&](auto tdx) {
        auto k = dsa::rows::rtd_bwd_kernel<decltype(nc)::value, typename decltype(tx)::type, typename decltype(tdx)::type>;
        hipLaunchKernelGGL(k, dim3((unsigned)nb), dim3(256), 0, st, p);
      });
    });
  });
  if (launch_check("rtd_bwd_kernel")) return 1;
  const int64_t off_w[1] = {0}, off_b[1] = {a->C};
  void* const out_w[1] = {a->dw};
  void* const out_b[1] = {a->db};
  if (reduce_cols(p.part, nb, a->C + 1, a->C, 1, off_w, out_w, a->param_dtype, st)) return 1;
  return a->db ? reduce_cols(p.part, nb, a->C + 1, 1, 1, off_b, out_b, a->param_dtype, st) : 0;
}

}  // extern "C"
