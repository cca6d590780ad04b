// dsa_common.h — shared device helpers for the fused disentangled-attention
// kernels (gfx950 / CDNA4).
//
// Matrix products use the 16x16 MFMA shapes:
//   bf16: v_mfma_f32_16x16x32_bf16  (A,B: 8 bf16 per lane, C: 4 fp32 per lane)
//   fp32: v_mfma_f32_16x16x4_f32    (A,B: 1 fp32 per lane, C: 4 fp32 per lane)
//
// Lane l of a wave is addressed as (c16 = l % 16, g = l / 16).  For a
// 16(M) x 16(N) x K product:
//   A fragment: row m = c16, a set of K indices chosen by g
//   B fragment: col n = c16, the same set of K indices chosen by g
//   C/D:        col n = c16, rows m = 4*g + e for e = 0..3
// Only the pairing of A and B k-indices matters for the result, so every
// product here picks a "k-set" per (step s, group g) and loads both operands
// with it:
//   CONTIG (bf16): k = 32*s + 8*g + [0..7]          -> one 16-byte load
//   ACC    (bf16): k = 32*s + 4*g + [0..3]  and  32*s + 16 + 4*g + [0..3]
//   (fp32)       : k = 16*s + 4*g + [0..3], four K=4 MFMAs per step
// The ACC set is exactly what a lane holds of two vertically adjacent C
// tiles, so a C tile (e.g. probabilities P) can be fed straight back into the
// next product as a B operand without a trip through LDS.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dsa {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

#define DSA_DEV __device__ __forceinline__

template <typename T>
struct Mfma;

template <>
struct Mfma<bf16> {
  static constexpr int KSTEP = 32;  // k indices consumed per step
  static constexpr int ACC_TILES_PER_STEP = 2;
  typedef bf16x8 frag;
  static DSA_DEV f32x4 mma(const frag& a, const frag& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  static DSA_DEV frag zero() {
    frag z;
#pragma unroll
    for (int e = 0; e < 8; ++e) z[e] = (bf16)0.0f;
    return z;
  }
  // CONTIG k-set from a contiguous row (row points at k = 0).
  static DSA_DEV frag load_contig(const bf16* row, int s, int g) {
    return *reinterpret_cast<const bf16x8*>(row + 32 * s + 8 * g);
  }
  // ACC k-set from a contiguous row.
  static DSA_DEV frag load_acc(const bf16* row, int s, int g) {
    bf16x4 lo = *reinterpret_cast<const bf16x4*>(row + 32 * s + 4 * g);
    bf16x4 hi = *reinterpret_cast<const bf16x4*>(row + 32 * s + 16 + 4 * g);
    frag f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      f[e] = lo[e];
      f[4 + e] = hi[e];
    }
    return f;
  }
  // ACC k-set from C tiles: tiles[2s] and tiles[2s+1] hold rows 4g+e.
  static DSA_DEV frag from_acc(const f32x4* tiles, int s) {
    frag f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      f[e] = (bf16)tiles[2 * s][e];
      f[4 + e] = (bf16)tiles[2 * s + 1][e];
    }
    return f;
  }
  // ACC k-set from 8 fp32 values gathered in k order (lo 4, hi 4).
  static DSA_DEV frag from_f32(const float* v) {
    frag f;
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = (bf16)v[e];
    return f;
  }
  // element index within the ACC k-set -> k offset inside the step
  static DSA_DEV int acc_k(int g, int e) { return (e < 4) ? (4 * g + e) : (16 + 4 * g + (e - 4)); }
  static constexpr int FRAG_ELEMS = 8;
};

template <>
struct Mfma<float> {
  static constexpr int KSTEP = 16;
  static constexpr int ACC_TILES_PER_STEP = 1;
  typedef f32x4 frag;
  static DSA_DEV f32x4 mma(const frag& a, const frag& b, f32x4 c) {
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[0], b[0], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[1], b[1], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[2], b[2], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[3], b[3], c, 0, 0, 0);
    return c;
  }
  static DSA_DEV frag zero() { return f32x4{0.f, 0.f, 0.f, 0.f}; }
  static DSA_DEV frag load_contig(const float* row, int s, int g) {
    return *reinterpret_cast<const f32x4*>(row + 16 * s + 4 * g);
  }
  static DSA_DEV frag load_acc(const float* row, int s, int g) { return load_contig(row, s, g); }
  static DSA_DEV frag from_acc(const f32x4* tiles, int s) { return tiles[s]; }
  static DSA_DEV frag from_f32(const float* v) { return f32x4{v[0], v[1], v[2], v[3]}; }
  static DSA_DEV int acc_k(int g, int e) { return 4 * g + e; }
  static constexpr int FRAG_ELEMS = 4;
};

DSA_DEV f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

template <typename T>
DSA_DEV float to_f32(T x) { return (float)x; }

template <typename T>
DSA_DEV T from_f32(float x) { return (T)x; }

// Cross-lane reductions over the 4 lanes that share c16 (lanes l, l^16,
// l^32, l^48): these hold the 4 row-groups of one C-tile column.
DSA_DEV float col_max(float x) {
  x = fmaxf(x, __shfl_xor(x, 16));
  x = fmaxf(x, __shfl_xor(x, 32));
  return x;
}
DSA_DEV float col_sum(float x) {
  x += __shfl_xor(x, 16);
  x += __shfl_xor(x, 32);
  return x;
}
DSA_DEV int wave_min(int x) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) x = min(x, __shfl_xor(x, o));
  return x;
}
DSA_DEV int wave_max(int x) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) x = max(x, __shfl_xor(x, o));
  return x;
}
DSA_DEV int wave_and(int x) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) x = x & __shfl_xor(x, o);
  return x;
}

// Stream compaction within a wave: the lanes with keep set store value at
// list[n + (their rank among those lanes)], in lane order; returns the new
// count, the same in every lane.  Callers order the LDS writes against
// later reads themselves.
template <typename V>
DSA_DEV int wave_append(bool keep, V value, V* list, int n) {
  const unsigned long long m = __ballot(keep);
  const int lane = __lane_id();
  if (keep) list[n + __popcll(m & ((1ull << lane) - 1ull))] = value;
  return n + __popcll(m);
}

// Orders LDS traffic between lanes of one wave (write by one lane, read by
// another).  DS instructions of a wave complete in order; this keeps the
// compiler from moving loads across the point.
DSA_DEV void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// c2p / p2c rows from a clamped relative position tc in [-A, A]
// (deberta_v2_native.py:395 / :407 and :488 / :503).
DSA_DEV int c2p_row(int tc, int A) { return min(max(tc + A, 0), 2 * A - 1); }
DSA_DEV int p2c_row(int tc, int A) { return min(max(-tc + A, 0), 2 * A - 1); }

// Transposed LDS reads (gfx950 ds_read_b64_tr_b16).  Within each 16-lane
// group, lane t receives element (t % 4) of the 8-byte chunks addressed by
// lanes 4*e + t/4 (e = 0..3).  So when lane c16 addresses
// X[k0 + c16/4][m0 + 4*(c16 % 4)] of a row-major array X, it receives
// X[k0 + e][m0 + c16] for e = 0..3: four consecutive k of column m0 + c16,
// i.e. half an MFMA operand fragment of the transposed tile.
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4_tr;
DSA_DEV bf16x4 tr4(const bf16* X, int str, int k0, int m0, int c16) {
  const bf16* p = X + (k0 + (c16 >> 2)) * str + m0 + 4 * (c16 & 3);
  bf16x4_tr v = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((__attribute__((address_space(3))) bf16x4_tr*)p);
  return __builtin_bit_cast(bf16x4, v);
}
DSA_DEV f32x4 tr4(const float* X, int str, int k0, int m0, int c16) {
  return f32x4{X[k0 * str + m0 + c16], X[(k0 + 1) * str + m0 + c16], X[(k0 + 2) * str + m0 + c16],
               X[(k0 + 3) * str + m0 + c16]};
}

// Eight elements of type T from two four-element vectors (a, then b).
template <typename T, typename V4>
DSA_DEV auto join_halves(const V4& a, const V4& b) {
  typedef T v8 __attribute__((ext_vector_type(8)));
  v8 r;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    r[e] = a[e];
    r[4 + e] = b[e];
  }
  return r;
}

DSA_DEV bf16x8 join8(bf16x4 a, bf16x4 b) {
  bf16x8 f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    f[e] = a[e];
    f[4 + e] = b[e];
  }
  return f;
}

// FE consecutive LDS elements starting at an element (not 16-byte) aligned
// address.  A 16-byte read at such an address is served far more slowly
// than aligned reads, so 16-bit elements are read as the FE/2 + 1 dwords
// that cover them (two-dword reads at the dword-aligned address below) and
// shifted into place with v_alignbit (by 16 bits when the address is odd in
// 16-bit units); 32-bit elements are read one by one.
template <typename T, int FE, typename F>
DSA_DEV void lds_read_elems(F& f, const T* p) {
  if constexpr (sizeof(T) == 2) {
    typedef const __attribute__((address_space(3))) unsigned* lds_u32;
    const uintptr_t a = (uintptr_t)p;
    const lds_u32 q = (lds_u32)(a & ~(uintptr_t)3);
    unsigned d[FE / 2 + 1];
#pragma unroll
    for (int k = 0; k < FE / 2 + 1; ++k) d[k] = q[k];
    const unsigned sh = (a & 2) ? 16u : 0u;
    typedef unsigned u_n __attribute__((ext_vector_type(FE / 2)));
    u_n r;
#pragma unroll
    for (int k = 0; k < FE / 2; ++k) r[k] = __builtin_amdgcn_alignbit(d[k + 1], d[k], sh);
    f = __builtin_bit_cast(F, r);
  } else {
#pragma unroll
    for (int e = 0; e < FE; ++e) f[e] = *(volatile const __attribute__((address_space(3))) T*)(p + e);
  }
}

// ds_read_b64_tr_b16 at an address the caller computed (see tr4).
DSA_DEV bf16x4 tr4_at(const bf16* p) {
  bf16x4_tr v = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((__attribute__((address_space(3))) bf16x4_tr*)p);
  return __builtin_bit_cast(bf16x4, v);
}

// 16-byte copy global -> LDS without registers (gfx950 global_load_lds_dwordx4):
// lane l of the wave writes lds_wave + 16 * l, where lds_wave is the same for
// every lane of the wave.  Completion is tracked by vmcnt only, and the
// caller waits for it explicitly (lds_dma_wait, vm_wait): the copy is
// issued from inline assembly because the compiler, which cannot tell which
// LDS bytes a copy writes, would otherwise wait for every outstanding copy
// before each LDS read, including reads of other buffers.
DSA_DEV void lds_dma16(const void* src, void* lds_wave) {
  const unsigned lds =
      __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)(__attribute__((address_space(3))) void*)lds_wave);
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds) : "memory", "m0");
}
// The same copy with the non-temporal hint, for data read once (the
// backward's pass over the saved relative term): the stream of it does not
// displace reused lines from the caches.
DSA_DEV void lds_dma16_nt(const void* src, void* lds_wave) {
  const unsigned lds =
      __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)(__attribute__((address_space(3))) void*)lds_wave);
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(src), "s"(lds) : "memory", "m0");
}
// Waits until at most N of this wave's vector-memory instructions are
// outstanding (they complete in issue order).
template <int N>
DSA_DEV void vm_wait() {
  static_assert(N >= 0 && N < 16, "vmcnt field");
  __builtin_amdgcn_s_waitcnt(0x0F70 | N);  // vmcnt(N), expcnt and lgkmcnt not waited for
}
// Waits for all of this wave's outstanding global loads, the LDS copies included.
DSA_DEV void lds_dma_wait() { vm_wait<0>(); }

// Row-major LDS tile with COLS elements per row whose 16-byte chunks are
// XOR-swizzled by row (chunk c of row r stored at chunk c ^ (r % CPR)), so that
// column reads across rows and row reads across lanes spread over the banks
// without padding.  Filled with lds_dma16, which writes 16-byte chunks in
// lane order.
template <typename T, int COLS>
struct Swz {
  static constexpr int VEC = 16 / sizeof(T);
  static constexpr int CPR = COLS / VEC;
  static_assert((CPR & (CPR - 1)) == 0, "chunks per row must be a power of two");
  DSA_DEV static int off(int r, int c) { return r * COLS + (((c / VEC) ^ (r & (CPR - 1))) * VEC) + (c % VEC); }
  // CONTIG k-set of row r (k = KSTEP*s + FE*g + [0, FE)) as an operand fragment
  DSA_DEV static typename Mfma<T>::frag row_frag(const T* X, int r, int s, int g) {
    constexpr int FE = Mfma<T>::FRAG_ELEMS;
    return *reinterpret_cast<const typename Mfma<T>::frag*>(X + off(r, Mfma<T>::KSTEP * s + FE * g));
  }
  // four consecutive rows k0 + e of column m0 + c16 (as tr4)
  DSA_DEV static f32x4 col4_f32(const float* X, int k0, int m0, int c16) {
    return f32x4{X[off(k0, m0 + c16)], X[off(k0 + 1, m0 + c16)], X[off(k0 + 2, m0 + c16)], X[off(k0 + 3, m0 + c16)]};
  }
  // ACC k-set of column m0 + c16 read transposed (as tr_acc)
  DSA_DEV static typename Mfma<T>::frag col_acc(const T* X, int k0, int m0, int g, int c16) {
    if constexpr (sizeof(T) == 2) {
      const int r0 = k0 + 4 * g + (c16 >> 2), r1 = r0 + 16, c = m0 + 4 * (c16 & 3);
      return join8(tr4_at(reinterpret_cast<const bf16*>(X) + off(r0, c)),
                   tr4_at(reinterpret_cast<const bf16*>(X) + off(r1, c)));
    } else {
      return col4_f32(reinterpret_cast<const float*>(X), k0 + 4 * g, m0, c16);
    }
  }
};

// Four consecutive rows k0 + e (e = 0..3) of column m0 + c16 of a row-major
// LDS array X as fp32, for 16-bit (fp16 / bf16) or fp32 elements.
template <typename B>
DSA_DEV f32x4 tr4_f32(const B* X, int str, int k0, int m0, int c16) {
  if constexpr (sizeof(B) == 2) {
    typedef B b4 __attribute__((ext_vector_type(4)));
    const bf16x4 r = tr4(reinterpret_cast<const bf16*>(X), str, k0, m0, c16);
    const b4 v = __builtin_bit_cast(b4, r);
    return f32x4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
  } else {
    return tr4(X, str, k0, m0, c16);
  }
}

// Operand fragment of column m0 + c16 of a row-major LDS array X whose rows
// are the k index: the CONTIG k-set (k = k0 + 8g + [0..7] for bf16,
// k0 + 4g + [0..3] for fp32), or the ACC k-set (k0 + 4g + [0..3] and
// k0 + 16 + 4g + [0..3] for bf16).
template <typename T>
DSA_DEV typename Mfma<T>::frag tr_contig(const T* X, int str, int k0, int m0, int g, int c16) {
  if constexpr (sizeof(T) == 2) {
    return join8(tr4(X, str, k0 + 8 * g, m0, c16), tr4(X, str, k0 + 8 * g + 4, m0, c16));
  } else {
    return tr4(X, str, k0 + 4 * g, m0, c16);
  }
}
template <typename T>
DSA_DEV typename Mfma<T>::frag tr_acc(const T* X, int str, int k0, int m0, int g, int c16) {
  if constexpr (sizeof(T) == 2) {
    return join8(tr4(X, str, k0 + 4 * g, m0, c16), tr4(X, str, k0 + 16 + 4 * g, m0, c16));
  } else {
    return tr4(X, str, k0 + 4 * g, m0, c16);
  }
}

// Workgroups are dispatched to the 8 XCDs in turn (workgroup n to XCD
// n % 8), and each XCD has its own L2.  xcd_remap gives workgroup n of a
// G-workgroup 1-D grid the logical index that makes each XCD run one
// contiguous range of logical indices, in order, so workgroups that are
// neighbours in logical order (the tiles of one batch and head, which read
// the same K/V or Q/dO) run on one XCD at about the same time and share its
// L2.  A bijection on [0, G).
DSA_DEV int xcd_remap(int n, int G) {
  constexpr int NX = 8;
  const int per = G / NX;
  return n < per * NX ? (n % NX) * per + n / NX : n;
}

// 1.0f that the compiler cannot see through: fma(fp16 -> fp32 x, one, y)
// then stays one mixed-precision FMA (v_fma_mix_f32) instead of being
// folded into a conversion and an add.
DSA_DEV float opaque_one() {
  float one;
  asm volatile("v_mov_b32 %0, 1.0" : "=v"(one));
  return one;
}

// a if C else b, for arrays and other objects a ternary cannot pick
template <bool C, typename X>
DSA_DEV const X& pick(const X& a, const X& b) {
  if constexpr (C) return a;
  else return b;
}

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

enum MaskMode { MASK_NONE = 0, MASK_KEY = 1, MASK_PAIR = 2, MASK_SEG = 3 };

}  // namespace dsa
