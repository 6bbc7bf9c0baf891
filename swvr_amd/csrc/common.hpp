// Shared device building blocks for the gfx950 readout kernels.
//
// Matrix products use the CDNA4 32x32 MFMA with fp32 accumulation:
//   bf16 / f16 : v_mfma_f32_32x32x16_{bf16,f16}   (8 operand elements per lane)
//   f32        : 8 x v_mfma_f32_32x32x2f32         (same per-lane operand vector)
// so every operand is handled as an 8-element vector per lane, whatever the
// dtype ("k16 step").
//
// Lane layout of one 32x32 block (wave of 64 lanes, lane = l):
//   A operand: row  l%32, reduction index block (l/32) -> 8 values
//   B operand: col  l%32, reduction index block (l/32) -> 8 values
//   C/D      : col  l%32, rows (r/4)*8 + (l/32)*4 + r%4 for register r = 0..15
// The reduction index of element t in lane-half (l/32) is the same function
// for A and B, so any permutation of the reduction index that is applied to
// both operands leaves the product unchanged.  The kernels use that to feed a
// product straight from another product's accumulator registers.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace swvr {

typedef __bf16 bf16_t;
typedef _Float16 f16_t;

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8_t;
typedef __attribute__((__vector_size__(8 * sizeof(float)))) float f32x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;

enum { kBF16 = 0, kF16 = 1, kF32 = 2 };

template <class T> struct Vec8;
template <> struct Vec8<bf16_t> { typedef bf16x8_t type; };
template <> struct Vec8<f16_t> { typedef f16x8_t type; };
template <> struct Vec8<float> { typedef f32x8_t type; };

constexpr float kNegInf = -__builtin_huge_valf();
constexpr float kPosInf = __builtin_huge_valf();
constexpr float kLog2e = 1.4426950408889634f;

constexpr int kThreads = 256;  // every kernel here runs 4 waves of 64 lanes

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

// One k16 step of C += A * B on a 32x32 block.
__device__ __forceinline__ void mfma_k16(f32x16_t& c, bf16x8_t a, bf16x8_t b) {
  c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ void mfma_k16(f32x16_t& c, f16x8_t a, f16x8_t b) {
  c = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ void mfma_k16(f32x16_t& c, f32x8_t a, f32x8_t b) {
#pragma unroll
  for (int t = 0; t < 8; ++t) c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[t], b[t], c, 0, 0, 0);
}

__device__ __forceinline__ f32x16_t zero16() {
  f32x16_t z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// exp(x) as 2^(x*log2 e) on the hardware exp2 (v_exp_f32).  exp(-inf) = 0.
__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }

template <class T> __device__ __forceinline__ T from_float(float x) { return (T)x; }
template <class T> __device__ __forceinline__ float to_float(T x) { return (float)x; }

// Row of the C/D block held by register r of this lane.
__device__ __forceinline__ int c_row(int r, int lane) { return (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3); }

// Stride (elements) of one operand row in LDS: BK plus 16 bytes of padding,
// which spreads the 32 rows a ds_read_b128 touches over all banks.
template <class T, int BK> struct LdsRow { static constexpr int value = BK + 16 / (int)sizeof(T); };

// ----------------------------------------------------------------------------
// Operand tiles staged global -> registers -> LDS.  LDS always holds a tile as
// [row][k] with k contiguous (stride LdsRow), which is what the MFMA operand
// reads want.  Global memory may hold it either way:
//   KTile: element (r, k) at base[r * ld + k]   (reduction index contiguous)
//   RTile: element (r, k) at base[k * ld + r]   (row index contiguous); the
//          tile is transposed in registers (8x8-byte blocks) on its way to LDS.
// Rows >= rows_valid and k >= k_valid read as zero.  k_valid is a multiple of
// 16 bytes worth of elements for KTile (the host checks K % 8 == 0) and rows of
// an RTile come in groups of 8 bytes (row counts are multiples of 8).
// ----------------------------------------------------------------------------
template <class T, int R, int BK>
struct KTile {
  static constexpr int CE = 16 / (int)sizeof(T);  // elements per 16-byte chunk
  static constexpr int CPR = BK / CE;             // chunks per row
  static constexpr int TOTAL = R * CPR;
  static constexpr int NCH = (TOTAL + kThreads - 1) / kThreads;
  static constexpr int LDR = LdsRow<T, BK>::value;
  uint4 v[NCH];
  const T* base;
  int64_t ld;
  int rows_valid;
  int k_valid;

  __device__ __forceinline__ void load(int k0) {
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = i * kThreads + (int)threadIdx.x;
      const int r = c / CPR, kc = (c % CPR) * CE;
      const bool ok = (TOTAL % kThreads == 0 || c < TOTAL) && r < rows_valid && k0 + kc < k_valid;
      v[i] = ok ? *reinterpret_cast<const uint4*>(base + (int64_t)r * ld + (k0 + kc)) : make_uint4(0, 0, 0, 0);
    }
  }
  __device__ __forceinline__ void store(T* lds) const {
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = i * kThreads + (int)threadIdx.x;
      if (TOTAL % kThreads == 0 || c < TOTAL) {
        const int r = c / CPR, kc = (c % CPR) * CE;
        *reinterpret_cast<uint4*>(lds + r * LDR + kc) = v[i];
      }
    }
  }
};

template <class T, int R, int BK>
struct RTile {
  static constexpr int RB = 8 / (int)sizeof(T);  // rows per 8-byte block
  static constexpr int NRB = R / RB;
  static constexpr int TOTAL = (BK / 8) * NRB;   // 8(k) x RB(r) blocks
  static constexpr int NB = (TOTAL + kThreads - 1) / kThreads;
  static constexpr int LDR = LdsRow<T, BK>::value;
  uint2 v[NB][8];
  const T* base;
  int64_t ld;
  int rows_valid;
  int k_valid;

  __device__ __forceinline__ void load(int k0) {
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int b = i * kThreads + (int)threadIdx.x;
      const int rb = b % NRB, kb = b / NRB;
      const int r = rb * RB;
      const bool okb = (TOTAL % kThreads == 0 || b < TOTAL) && r < rows_valid;
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        const int k = k0 + kb * 8 + kk;
        v[i][kk] = (okb && k < k_valid) ? *reinterpret_cast<const uint2*>(base + (int64_t)k * ld + r)
                                        : make_uint2(0, 0);
      }
    }
  }
  __device__ __forceinline__ void store(T* lds) const {
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int b = i * kThreads + (int)threadIdx.x;
      if (!(TOTAL % kThreads == 0 || b < TOTAL)) continue;
      const int rb = b % NRB, kb = b / NRB;
      const int r = rb * RB;
      if constexpr (sizeof(T) == 2) {
        // 8 k-rows x 4 elements -> 4 rows x 8 k-values (16 bytes each)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          // element j of a k-row is the low (j even) or high (j odd) half of
          // word x (j < 2) or y (j >= 2); pair k-rows 2p, 2p+1 into one word
          uint32_t w[8];
#pragma unroll
          for (int kk = 0; kk < 8; ++kk) w[kk] = (j < 2) ? v[i][kk].x : v[i][kk].y;
          uint32_t o[4];
#pragma unroll
          for (int p = 0; p < 4; ++p)
            o[p] = (j & 1) ? ((w[2 * p] >> 16) | (w[2 * p + 1] & 0xffff0000u))
                           : ((w[2 * p] & 0xffffu) | (w[2 * p + 1] << 16));
          *reinterpret_cast<uint4*>(lds + (r + j) * LDR + kb * 8) = make_uint4(o[0], o[1], o[2], o[3]);
        }
      } else {
        // 8 k-rows x 2 floats -> 2 rows x 8 k-values (32 bytes each)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          uint4 o0, o1;
          o0.x = j ? v[i][0].y : v[i][0].x;
          o0.y = j ? v[i][1].y : v[i][1].x;
          o0.z = j ? v[i][2].y : v[i][2].x;
          o0.w = j ? v[i][3].y : v[i][3].x;
          o1.x = j ? v[i][4].y : v[i][4].x;
          o1.y = j ? v[i][5].y : v[i][5].x;
          o1.z = j ? v[i][6].y : v[i][6].x;
          o1.w = j ? v[i][7].y : v[i][7].x;
          uint4* dst = reinterpret_cast<uint4*>(lds + (r + j) * LDR + kb * 8);
          dst[0] = o0;
          dst[1] = o1;
        }
      }
    }
  }
};

// One LDS stage of C[FM][FN] += A_tile * B_tile^T for this wave: A rows
// a_row0 .. a_row0 + 32*FM, B rows b_row0 .. b_row0 + 32*FN, BK reduction.
template <class T, int BK, int FM, int FN>
__device__ __forceinline__ void stage_mma(f32x16_t (&acc)[FM][FN], const T* sA, const T* sB, int a_row0,
                                          int b_row0) {
  typedef typename Vec8<T>::type V8;
  constexpr int LDR = LdsRow<T, BK>::value;
  const int lane = lane_id();
  const int lr = lane & 31, lk = (lane >> 5) * 8;
#pragma unroll
  for (int j = 0; j < BK / 16; ++j) {
    V8 a[FM], b[FN];
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
      a[fm] = *reinterpret_cast<const V8*>(sA + (a_row0 + fm * 32 + lr) * LDR + j * 16 + lk);
#pragma unroll
    for (int fn = 0; fn < FN; ++fn)
      b[fn] = *reinterpret_cast<const V8*>(sB + (b_row0 + fn * 32 + lr) * LDR + j * 16 + lk);
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) mfma_k16(acc[fm][fn], a[fm], b[fn]);
  }
}

// Double-buffered reduction loop: acc += A[rows, 0:Kred] * B[rows, 0:Kred]^T.
// `side` is called as side.pre(kt) before the stage's products (issue extra
// global loads) and side.post(kt) after them (store those loads to LDS); all
// threads pass a barrier after every stage, so side data written in stage kt
// is visible from stage kt+1 on.  Ends with a barrier.
template <class T, int BK, int FM, int FN, class TA, class TB, class Side>
__device__ __forceinline__ void reduce_loop(f32x16_t (&acc)[FM][FN], TA& ta, TB& tb, T* sA0, T* sA1, T* sB0,
                                            T* sB1, int k_total, int a_row0, int b_row0, Side& side) {
  const int nk = (k_total + BK - 1) / BK;
  if (nk > 0) {
    ta.load(0);
    tb.load(0);
    ta.store(sA0);
    tb.store(sB0);
  }
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const bool odd = kt & 1;
    const T* cA = odd ? sA1 : sA0;
    const T* cB = odd ? sB1 : sB0;
    const bool more = kt + 1 < nk;
    if (more) {
      ta.load((kt + 1) * BK);
      tb.load((kt + 1) * BK);
    }
    side.pre(kt);
    stage_mma<T, BK, FM, FN>(acc, cA, cB, a_row0, b_row0);
    if (more) {
      ta.store(odd ? sA0 : sA1);
      tb.store(odd ? sB0 : sB1);
    }
    side.post(kt);
    __syncthreads();
  }
}

struct NoSide {
  __device__ __forceinline__ void pre(int) {}
  __device__ __forceinline__ void post(int) {}
};

// blockIdx -> tile index such that each XCD (blocks are dealt to the 8 XCDs
// round-robin) works through a contiguous range of tile indices, so the tiles
// that run together on one XCD share operands in that XCD's L2.
__device__ __forceinline__ int xcd_swizzle(int b, int n) {
  constexpr int X = 8;
  const int q = n / X;
  if (b >= q * X) return b;
  return (b % X) * q + b / X;
}

__device__ __forceinline__ float wave_max32(float x) { return fmaxf(x, __shfl_xor(x, 32)); }
__device__ __forceinline__ float wave_sum32(float x) { return x + __shfl_xor(x, 32); }

}  // namespace swvr
