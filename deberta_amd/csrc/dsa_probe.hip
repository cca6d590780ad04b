// dsa_probe.hip — libdsa_probe.so (include/dsa_probe.h): a bf16 MFMA
// throughput probe, the measured counterpart of the published dense peak.
#include <hip/hip_runtime.h>

#include "../../include/dsa_probe.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// Four independent accumulation chains of the 32x32x16 bf16 product per
// wave (32768 flops each) keep the matrix pipe busy without waiting on a
// result; launched with eight workgroups of four waves per CU, each SIMD
// holds eight waves.  (The 16x16x32 form needs about sixteen chains in
// flight per SIMD to come near the same rate.)
__global__ __launch_bounds__(256) void mfma_bf16_probe(float* sink, int iters) {
  bf16x8 a, b;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    a[e] = (__bf16)(1.0f + 1e-3f * (float)((threadIdx.x + e) & 7));
    b[e] = (__bf16)(1.0f - 1e-3f * (float)((threadIdx.x * 3 + e) & 7));
  }
  f32x16 c[4];
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int e = 0; e < 16; ++e) c[u][e] = 0.f;
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int u = 0; u < 4; ++u) c[u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c[u], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int e = 0; e < 16; ++e) s += c[u][e];
  sink[(size_t)blockIdx.x * 256 + threadIdx.x] = s;
}

// The table-gradient traffic a backward without a dS workspace would make:
// one workgroup per (b, h, 128-key tile), which meets the L + 127 offsets
// d = i - j of its keys and all L queries, adds one fp32 row of 64 values
// (D = 64) per offset and per kind (c2p, p2c) into per-head accumulators
// [H][2][nrows][64] (row d + LkP - 1), after summing its four waves:
// global_atomic_add_f32, one row of 64 consecutive floats per wave
// instruction.  The added values are ones (the rate, not the sums, is
// measured).
__global__ __launch_bounds__(256) void dsfree_flush_probe(float* acc, int H, int NKT, int L, int nrows) {
  const int w = blockIdx.x;
  const int kt = w % NKT, h = (w / NKT) % H;
  const int d_lo = -(kt * 128 + 127), n = L + 127;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int LkP = NKT * 128;
  for (int kind = 0; kind < 2; ++kind) {
    float* base = acc + (size_t)(h * 2 + kind) * nrows * 64;
    for (int r = wave; r < n; r += 4) {
      const int row = d_lo + r + LkP - 1;
      if (row >= 0 && row < nrows) unsafeAtomicAdd(base + (size_t)row * 64 + lane, 1.0f);
    }
  }
}

}  // namespace

extern "C" int dsa_probe_dsfree_flush(int B, int H, int L, float* acc, void* stream) {
  if (B < 1 || H < 1 || L < 1 || L % 128 || !acc) return 1;
  const int NKT = L / 128;
  hipLaunchKernelGGL(dsfree_flush_probe, dim3((unsigned)(B * H * NKT)), dim3(256), 0, static_cast<hipStream_t>(stream),
                     acc, H, NKT, L, 2 * L);
  return hipGetLastError() == hipSuccess ? 0 : 1;
}

extern "C" int dsa_probe_mfma_bf16(int workgroups, int iters, float* sink, void* stream) {
  if (workgroups < 1 || iters < 1 || !sink) return 1;
  hipLaunchKernelGGL(mfma_bf16_probe, dim3((unsigned)workgroups), dim3(256), 0, static_cast<hipStream_t>(stream), sink,
                     iters);
  return hipGetLastError() == hipSuccess ? 0 : 1;
}
