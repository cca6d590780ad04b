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
//   dsa_order_cost_kernel  one block per batch row: the segment range of
//                          every 32-token chunk (in LDS), then per tile the
//                          number of tiles of the other side whose ranges
//                          meet its own, plus one (ChunkRange::meets, the
//                          tile test of the kernels themselves, on ranges)
//   dsa_order_sort_kernel  one block: a counting sort of the (batch row,
//                          tile) items by cost, heaviest first
//
// The kernels then map workgroup r to item order[r / H] and head r % H.
// The order among items of equal cost depends on the atomics' timing; each
// workgroup writes only its own outputs, so the results do not.
#pragma once

#include "dsa_tiles.h"

namespace dsa {

struct OrderParams {
  FwdParams f;
  int* cost;    // [B * ntiles]
  int* order;   // [B * ntiles]
  int ntiles;   // tiles per batch row
  int fwd;      // 1: forward query tiles (128) against 64-key tiles; 0: dkdv key tiles (128) against 32-query chunks
};

constexpr int ORDER_MAX_CHUNKS = 1024;  // 32-token chunks (L <= 32768)
constexpr int ORDER_MAX_COST = 1025;    // tiles of the other side + 1

__global__ __launch_bounds__(256) void dsa_order_cost_kernel(OrderParams op) {
  const FwdParams& p = op.f;
  __shared__ int clo[ORDER_MAX_CHUNKS], chi[ORDER_MAX_CHUNKS];
  const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
  const int L = p.Lk;  // masks need Lq == Lk
  const int nch = (L + 31) / 32;
  // chunk ranges: half a wave per chunk, one token a lane
  for (int t0 = 0; t0 < nch * 32; t0 += 256) {
    const int t = t0 + tid;
    const int s = t < L ? seg_at(p, b, t) : 0;
    int lo = s != 0 ? s : 0x7fffffff, hi = s != 0 ? s : (int)0x80000000;
#pragma unroll
    for (int o = 1; o < 32; o <<= 1) {
      lo = min(lo, __shfl_xor(lo, o));
      hi = max(hi, __shfl_xor(hi, o));
    }
    if ((lane & 31) == 0 && t < nch * 32) {
      clo[t / 32] = lo;
      chi[t / 32] = hi;
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
  for (int i = tid; i < op.ntiles; i += 256) {
    int n = 1;
    if (op.fwd) {
      const ChunkRange q = range(4 * i, 4);
      for (int k = 0; 2 * k < nch; ++k) n += q.meets(range(2 * k, 2)) ? 1 : 0;
    } else {
      const ChunkRange kr = range(4 * i, 4);
      for (int c = 0; c < nch; ++c) n += kr.meets(range(c, 1)) ? 1 : 0;
    }
    op.cost[(int64_t)b * op.ntiles + i] = min(n, ORDER_MAX_COST);
  }
}

__global__ __launch_bounds__(1024) void dsa_order_sort_kernel(OrderParams op) {
  // cost c sits at position ORDER_MAX_COST - c (heaviest first); thread t
  // owns positions 2t and 2t + 1
  __shared__ int hist[2 * 1024];
  __shared__ int wsum[16];
  static_assert(ORDER_MAX_COST < 2 * 1024, "two positions a thread");
  const int n = op.f.B * op.ntiles, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  hist[2 * tid] = 0;
  hist[2 * tid + 1] = 0;
  __syncthreads();
  for (int i = tid; i < n; i += 1024) atomicAdd(&hist[ORDER_MAX_COST - op.cost[i]], 1);
  __syncthreads();
  // exclusive scan over the positions: pairs, then an inclusive scan within
  // the wave, then the wave totals
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
  for (int i = tid; i < n; i += 1024) op.order[atomicAdd(&hist[ORDER_MAX_COST - op.cost[i]], 1)] = i;
}

}  // namespace dsa
