// dsa_bwd_dqtab.h — the DQ and FOLD stages' main kernels in one launch
// (gfx950).
//
// Both only read dS (and Q, K, the gathered tables).  Launched as one grid,
// their workgroups share the CUs (two per CU, of either kind, over one LDS
// allocation sized for the larger of the two) with no stream fork and join
// around them: a fork to a second stream and the join back cost 7 to 13 us
// of idle GPU between the dkdv kernel and these two.
//
// Grid order: the table workgroups first (their count rounded up to a
// multiple of eight with empty workgroups), then the dq workgroups.  The
// table workgroups are the longer ones and start at once; the dq
// workgroups fill the remaining slots and the gaps the table kernel's
// uneven ends leave.  Workgroups go to the XCDs in turn (workgroup n to XCD
// n % 8), so with the rounding each kind's logical index keeps the
// remainder mod 8 of its physical one, which the kernels' XCD-aware orders
// (xcd_remap) rely on.  (Measured at B=32, L=512: 305 against 313 us for
// the backward with the two kernels on two streams; alternating the kinds
// in runs of eight took 350.)
#pragma once

#include "dsa_bwd_dq.h"
#include "dsa_bwd_table.h"

namespace dsa {

template <typename T, int D, bool LISTED, bool QC>
__global__ __launch_bounds__(256, 2) void dsa_bwd_dqtab_kernel(BwdParams bp, BwdParams tp, int ntab, int nt8, int ndq) {
  __shared__ union Lds {
    DqLds<T, D> dq;
    TabLds<T, D> tab;
  } L;
  const int n = blockIdx.x;
  if (n < nt8) {
    if (n < ntab) table_body<T, D, LISTED>(tp, n, ntab, L.tab);
  } else {
    dq_body<T, D, QC>(bp, n - nt8, ndq, L.dq);
  }
}

}  // namespace dsa
