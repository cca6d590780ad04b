// dsa_order.h — heaviest-first launch order under key-padding and segment
// masks (gfx950).
//
// Under such a mask the workgroups of the forward (one per batch row, head
// and 128-query tile) and of the dkdv kernel (one per batch row, head and
// 128-key tile) differ in work by the number of tiles they skip: a query
// tile inside a long document visits many key tiles, one inside a short
// document few.  Launched in (batch, head, tile) order, the heaviest
// workgroups can start last and stretch the launch.  These two small
// kernels give those launches an order with the heaviest tiles first:
//
//   dsa_order_cost_kernel  one block per (batch row, 4 tiles): the segment
//                          range of every 32-token chunk of the row (in
//                          LDS, from 16-byte loads), then one wave per
//                          tile counts the tiles of the other side whose
//                          ranges meet its own, plus one (ChunkRange::meets,
//                          the tile test of the kernels themselves, on
//                          ranges), the lanes over the other side's tiles
//   dsa_order_sort_kernel  one block: a counting sort of the (batch row,
//                          tile) items by cost, heaviest first
//
// The cost blocks also run inside other launches that precede the order's
// use: the forward's table copy (dsa_fwd_pre_kernel) and the backward's
// preparation (dsa_bwd_prep_kernel), so that only the sort is a launch of
// its own.
//
// Both take up to two orders at once (the backward's dkdv and dq orders):
// launches of a few microseconds each dominate at C4 sizes.
//
// The kernels then map workgroup r to item order[r / H] and head r % H.
// The order among items of equal cost depends on the atomics' timing; each
// workgroup writes only its own outputs, so the results do not.
#pragma once

#include "dsa_tiles.h"

namespace dsa {

constexpr int ORDER_MAX_CHUNKS = 1024;  // 32-token chunks (L <= 32768)
constexpr int ORDER_MAX_COST = 1025;    // tiles of the other side + 1

// Segment id of token t of batch row b (0: inactive), four tokens at a time
// from 16-byte loads when the row allows it.
DSA_DEV int4 seg4_at(const FwdParams& p, int b, int t, int L) {
  int4 s = {0, 0, 0, 0};
  if (p.seg) {
    const int32_t* row = p.seg + (int64_t)b * p.segb;
    if (t + 3 < L && ((reinterpret_cast<uintptr_t>(row + t) & 15) == 0)) return *reinterpret_cast<const int4*>(row + t);
    s.x = t < L ? row[t] : 0;
    s.y = t + 1 < L ? row[t + 1] : 0;
    s.z = t + 2 < L ? row[t + 2] : 0;
    s.w = t + 3 < L ? row[t + 3] : 0;
  } else {
    const uint8_t* row = p.kk + (int64_t)b * p.kkb;
    s.x = t < L ? row[t] != 0 : 0;
    s.y = t + 1 < L ? row[t + 1] != 0 : 0;
    s.z = t + 2 < L ? row[t + 2] != 0 : 0;
    s.w = t + 3 < L ? row[t + 3] != 0 : 0;
  }
  return s;
}

// Heaviest-first counting sort of n items by cost (in [1, ORDER_MAX_COST]),
// by one block of 1024 threads: order[k] = the k-th item.  cost may be in
// LDS or global memory; hist is 2 * 1024 ints of LDS, wsum 16.  Holds
// barriers: every thread of the block calls it.
template <typename C>
DSA_DEV void sort_by_cost(const C* cost, int n, int* order, int* hist, int* wsum) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  hist[2 * tid] = 0;
  hist[2 * tid + 1] = 0;
  __syncthreads();
  for (int i = tid; i < n; i += 1024) atomicAdd(&hist[ORDER_MAX_COST - cost[i]], 1);
  __syncthreads();
  const int a = hist[2 * tid], b = hist[2 * tid + 1];
  int x = a + b;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  if (lane == 63) wsum[w] = x;
  __syncthreads();
  int base = 0;
  for (int k = 0; k < w; ++k) base += wsum[k];
  const int start = base + x - (a + b);
  hist[2 * tid] = start;
  hist[2 * tid + 1] = start + a;
  __syncthreads();
  for (int i = tid; i < n; i += 1024) order[atomicAdd(&hist[ORDER_MAX_COST - cost[i]], 1)] = i;
  __syncthreads();
}

// One order of the fused kernel.
struct OrderJob {
  int* cost;   // [B * ntiles] (written too, for inspection)
  int* order;  // [B * ntiles]
  int ntiles;
  int fwd;
};
struct OrderParams2 {
  FwdParams f;
  OrderJob job[2];
  int njobs;
};

constexpr int ORDER_TPB = 4;  // tiles per cost block (one wave each)

// Cost block (batch row b, tiles 4 by .. 4 by + 3, job jb) of 256 threads.
// Holds a barrier: every thread of the block calls it.
DSA_DEV void order_cost_block(const OrderParams2& op2, int b, int by, int jb) {
  const FwdParams& p = op2.f;
  const OrderJob& op = op2.job[jb];
  __shared__ int clo[ORDER_MAX_CHUNKS], chi[ORDER_MAX_CHUNKS];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int L = p.Lk;  // masks need Lq == Lk
  const int nch = (L + 31) / 32;
  // chunk ranges: eight lanes per chunk, four tokens a lane; all of a
  // thread's loads are issued before the reductions
  constexpr int PER = 4;  // 4-token groups a thread takes per pass
  for (int g0 = 0; g0 < nch * 8; g0 += 256 * PER) {
    int4 s[PER];
#pragma unroll
    for (int u = 0; u < PER; ++u) s[u] = seg4_at(p, b, 4 * (g0 + 256 * u + tid), L);
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int g = g0 + 256 * u + tid;  // 4-token group; chunk g / 8
      int lo = 0x7fffffff, hi = (int)0x80000000;
      const int v[4] = {s[u].x, s[u].y, s[u].z, s[u].w};
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (v[e] != 0) {
          lo = min(lo, v[e]);
          hi = max(hi, v[e]);
        }
#pragma unroll
      for (int o = 1; o < 8; o <<= 1) {
        lo = min(lo, __shfl_xor(lo, o));
        hi = max(hi, __shfl_xor(hi, o));
      }
      if ((lane & 7) == 0 && g < nch * 8) {
        clo[g / 8] = lo;
        chi[g / 8] = hi;
      }
    }
  }
  __syncthreads();
  auto range = [&](int c0, int n) {  // union of chunks [c0, c0 + n)
    ChunkRange r{0x7fffffff, (int)0x80000000, 1};
    for (int c = c0; c < min(c0 + n, nch); ++c) {
      r.lo = min(r.lo, clo[c]);
      r.hi = max(r.hi, chi[c]);
    }
    return r;
  };
  const int i = by * ORDER_TPB + w;  // this wave's tile
  if (i >= op.ntiles) return;
  const ChunkRange mine = range(4 * i, 4);
  // the other side: 64-key tiles (two chunks) for the forward, 32-query
  // chunks for dkdv; one per lane per step
  const int per = op.fwd ? 2 : 1;
  const int nother = (nch + per - 1) / per;
  int n = 1;
  for (int u0 = 0; u0 < nother; u0 += 64) {
    const int u = u0 + lane;
    const bool hit = u < nother && mine.meets(range(per * u, per));
    n += __popcll(__ballot(hit));
  }
  if (lane == 0) op.cost[(int64_t)b * op.ntiles + i] = min(n, ORDER_MAX_COST);
}

__global__ __launch_bounds__(256) void dsa_order_cost_kernel(OrderParams2 op2) {
  order_cost_block(op2, blockIdx.x, blockIdx.y, blockIdx.z);
}

// The forward's preparation in one launch: its launch-order cost blocks
// (ncost of them, batch row fastest; none without an order) first, then the
// k-step copies of the relative tables (ncopy blocks per table; none
// without the copies).  The sort runs after it (dsa_order_sort_kernel).
__global__ __launch_bounds__(256) void dsa_fwd_pre_kernel(TableKs t, OrderParams2 op2, int ncost, int ncopy) {
  const int blk = blockIdx.x;
  if (blk < ncost) {
    order_cost_block(op2, blk % op2.f.B, blk / op2.f.B, 0);
  } else {
    const int k = blk - ncost;
    table_ks_block(t, k % ncopy, k / ncopy);
  }
}

__global__ __launch_bounds__(1024) void dsa_order_sort_kernel(OrderParams2 op) {
  // cost c sits at position ORDER_MAX_COST - c (heaviest first); thread t
  // owns positions 2t and 2t + 1
  __shared__ int hist[2 * 1024];
  __shared__ int wsum[16];
  static_assert(ORDER_MAX_COST < 2 * 1024, "two positions a thread");
  for (int j = 0; j < op.njobs; ++j) sort_by_cost(op.job[j].cost, op.f.B * op.job[j].ntiles, op.job[j].order, hist, wsum);
}

}  // namespace dsa
