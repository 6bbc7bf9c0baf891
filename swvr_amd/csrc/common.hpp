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

#include <type_traits>

namespace swvr {

typedef __bf16 bf16_t;
typedef _Float16 f16_t;

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8_t;
typedef __attribute__((__vector_size__(8 * sizeof(float)))) float f32x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;

enum { kBF16 = 0, kF16 = 1, kF32 = 2, kFP8 = 3 };  // kFP8: h, W in OCP e4m3; E in bf16

template <class T> struct Vec8;
template <> struct Vec8<bf16_t> { typedef bf16x8_t type; };
template <> struct Vec8<f16_t> { typedef f16x8_t type; };
template <> struct Vec8<float> { typedef f32x8_t type; };

constexpr float kNegInf = -__builtin_huge_valf();
constexpr float kPosInf = __builtin_huge_valf();
constexpr float kLog2e = 1.4426950408889634f;

constexpr int kThreads = 256;  // every kernel here runs 4 waves of 64 lanes

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
// Wave index in a 1-D workgroup: uniform across the wave, so it lives in a
// scalar register (every wave-derived address with it).
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

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

// A product whose B operand is taken from another product's C/D registers
// 8c..8c+7 (lane half hi) reduces over the rows 16c + 8(t/4) + 4hi + t%4,
// t = 0..7, of a 32-row block.  Operand tiles that feed such products store
// each group of 8 rows contiguously: position p of a packed tile holds row
// pe_row(p), so an operand is one 16-byte (two for fp32) LDS read at
// position 32 blk + 8 (2c + hi).
__host__ __device__ __forceinline__ int pe_row(int p) {
  const int blk = p >> 5, g = (p >> 3) & 3, i = p & 7;
  const int c = g >> 1, hi = g & 1;
  return blk * 32 + 16 * c + 8 * (i >> 2) + 4 * hi + (i & 3);
}

// ----------------------------------------------------------------------------
// Direct-to-LDS operand pipeline.
//
// Operand tiles move HBM -> LDS with buffer_load_dwordx4 ... lds: each lane
// names a 16-byte source chunk, the wave's 64 chunks land contiguously in LDS,
// and no registers are used, so the reduction loop keeps kStages-1 slices in
// flight.  A buffer resource whose range is 2^31-1 bytes turns any chunk the
// tile does not own (rows or k beyond the operand) into a zero fill: such a
// lane's offset is set to kOOB, past the range.
//
// LDS tile layouts (16-byte chunks, XOR-swizzled within a row so that the
// MFMA operand reads are free of bank conflicts):
//   KTile: [R rows][BK] elements, the reduction index contiguous in global
//          memory (element (r, k) at base[r * ld + k]); operand read = one
//          ds_read_b128 (bf16/f16) or two (f32) per lane.
//   RTile: [BK][R] elements, the row index contiguous in global memory
//          (element (r, k) at base[k * ld + r]); operand read transposes in
//          the LDS read: two ds_read_b64_tr_b16 per lane (bf16/f16), or eight
//          ds_read_b32 (f32).
// ----------------------------------------------------------------------------
typedef int rsrc_t __attribute__((ext_vector_type(4)));  // buffer descriptor (4 SGPRs)
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef short s16x8_t __attribute__((ext_vector_type(8)));

constexpr int kStages = 4;   // default LDS ring depth of the reduction loop
constexpr uint32_t kOOB = 0x80000000u;

// Reduction slice per stage: 32 elements (64-byte rows) for bf16 / f16, 16
// (64-byte rows) for f32, which keeps the four-stage ring inside LDS.
template <class T> struct SliceK { static constexpr int value = sizeof(T) == 2 ? 32 : 16; };

// XOR swizzle of the 16-byte chunks of an LDS row of `cpr` chunks.  The
// gfx950 LDS has 64 four-byte banks (256 bytes per cycle) and serves a
// ds_read_b128 sixteen consecutive lanes per cycle; the operand reads have
// those sixteen lanes on sixteen consecutive rows at the same logical chunk,
// so the sixteen rows must land on sixteen distinct 16-byte bank groups.
__device__ __forceinline__ int chunk_swizzle(int row, int cpr) {
  const int rows_per_256 = cpr >= 16 ? 1 : 16 / cpr;
  const int span = cpr >= 16 ? 16 : cpr;
  return (row / rows_per_256) % span;
}

// Raw buffer descriptor over [base, base + 2^31 - 1): stride 0, 32-bit data
// format (the CDNA descriptor's fourth dword); a null base gives an empty
// range, so every load through it returns zeros.  base must be wave-uniform.
__device__ __forceinline__ rsrc_t make_rsrc(const void* base) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  rsrc_t r;
  r.x = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  r.y = __builtin_amdgcn_readfirstlane((int)((a >> 32) & 0xFFFFu));
  r.z = base ? 0x7FFFFFFF : 0;
  r.w = 0x00020000;
  return r;
}

// The same descriptor as the compiler's buffer resource type, for the buffer
// load / store builtins (whose memory operations the compiler counts, unlike
// inline asm).  A load at offset kOOB returns zeros; a store there is dropped.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  const uint64_t ua = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32)) << 32) |
                      (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(ua), (short)0, base ? 0x7FFFFFFF : 0,
                                           0x00020000);
}

// Wave-uniform LDS byte address of a pointer into __shared__ memory.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(size_t)(__attribute__((address_space(3))) const char*)p);
}

// buffer_load_dwordx4 ... lds: one 16-byte chunk per lane into LDS; load i of
// a batch lands at lds + i * 4096 + 16 * lane (M0 holds the LDS base; it is
// saved and restored around the batch).  Issued from inline assembly so that
// the compiler does not guard every later LDS read with a wait for all
// outstanding loads: the reduction loops order these loads themselves
// (wait_stages + stage_barrier).  On this chip generation an LDS-DMA load
// that follows a scalar write of M0 needs one wait state, or it may take the
// previous M0 and write a wrong LDS address; the compiler inserts that wait
// for its own code but not inside assembly, hence the s_nop after each write.
// s_add_u32 on M0 also writes SCC, so the assembly declares SCC clobbered (the
// compiler may otherwise keep a comparison's result in SCC across the batch).
__device__ __forceinline__ void dma_batch1(rsrc_t r, uint32_t v0, uint32_t lds_any) {
  const uint32_t lds = __builtin_amdgcn_readfirstlane(lds_any);
  uint32_t save;
  asm volatile(
      "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %1, %2, 0 offen lds\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(save)
      : "v"(v0), "s"(r), "s"(lds)
      : "memory", "scc");
}
template <int STEP>
__device__ __forceinline__ void dma_batch2(rsrc_t r, uint32_t v0, uint32_t v1, uint32_t lds) {
  uint32_t save;
  asm volatile(
      "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %4\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %1, %3, 0 offen lds\n\t"
      "s_add_u32 m0, m0, %5\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %2, %3, 0 offen lds\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(save)
      : "v"(v0), "v"(v1), "s"(r), "s"(lds), "i"(STEP)
      : "memory", "scc");
}
template <int STEP>
__device__ __forceinline__ void dma_batch4(rsrc_t r, uint32_t v0, uint32_t v1, uint32_t v2, uint32_t v3,
                                           uint32_t lds) {
  uint32_t save;
  asm volatile(
      "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %6\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %1, %5, 0 offen lds\n\t"
      "s_add_u32 m0, m0, %7\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %2, %5, 0 offen lds\n\t"
      "s_add_u32 m0, m0, %7\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %3, %5, 0 offen lds\n\t"
      "s_add_u32 m0, m0, %7\n\ts_nop 0\n\t"
      "buffer_load_dwordx4 %4, %5, 0 offen lds\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(save)
      : "v"(v0), "v"(v1), "v"(v2), "v"(v3), "s"(r), "s"(lds), "i"(STEP)
      : "memory", "scc");
}
// NI loads of one thread, STEP bytes apart in LDS starting at lds.
template <int NI, int STEP>
__device__ __forceinline__ void dma_n(rsrc_t r, const uint32_t (&v)[NI], uint32_t lds_any) {
  const uint32_t lds = __builtin_amdgcn_readfirstlane(lds_any);  // wave-uniform by construction
  if constexpr (NI == 1) {
    dma_batch1(r, v[0], lds);
  } else if constexpr (NI == 2) {
    dma_batch2<STEP>(r, v[0], v[1], lds);
  } else {
    static_assert(NI % 4 == 0, "batches of 4");
#pragma unroll
    for (int i = 0; i < NI; i += 4) dma_batch4<STEP>(r, v[i], v[i + 1], v[i + 2], v[i + 3], lds + i * STEP);
  }
}

// s_waitcnt vmcnt(N) (gfx9 encoding; expcnt and lgkmcnt left unconstrained).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Workgroup barrier for the direct-to-LDS pipeline.  __syncthreads() carries a
// release fence that waits for every outstanding vector memory operation
// (vmcnt(0)), which would drain the whole prefetch ring; the stage data here
// is already covered by the explicit vmcnt wait that precedes the barrier, so
// only LDS traffic (lgkmcnt) is waited for.  The "memory" clobber keeps the
// compiler from moving memory accesses across it.
__device__ __forceinline__ void stage_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Compiler-only fence: keeps the scheduler from hoisting the LDS reads of a
// later epilogue block above this point (which would keep them all live).
__device__ __forceinline__ void sched_fence() { asm volatile("" ::: "memory"); }

// A zero the compiler cannot see through.  Added to LDS gather addresses in
// an epilogue, it stops loop-invariant code motion from hoisting dozens of
// gather addresses out of the tile loop and keeping them live (spills).
__device__ __forceinline__ int opaque_zero() {
  int z;
  asm volatile("v_mov_b32 %0, 0" : "=v"(z));
  return z;
}

// Wait until the next stage of an NS-deep ring has landed, when `ahead`
// stages (L loads per thread each) have been issued after it: at most
// min(ahead, NS - 2) stages may stay outstanding.
template <int L, int NS>
__device__ __forceinline__ void wait_stages(int ahead) {
  static_assert(NS >= 2 && NS <= 4, "ring depth");
  if constexpr (NS == 4) {
    if (ahead >= 2)
      wait_vmcnt<2 * L>();
    else if (ahead == 1)
      wait_vmcnt<L>();
    else
      wait_vmcnt<0>();
  } else if constexpr (NS == 3) {
    if (ahead >= 1)
      wait_vmcnt<L>();
    else
      wait_vmcnt<0>();
  } else {
    wait_vmcnt<0>();
  }
}

template <class T, int R, int BK, int NT = kThreads>
struct KTile {
  typedef KTile Layout;                             // LDS layout (operand reads)
  static constexpr int CE = 16 / (int)sizeof(T);    // elements per chunk
  static constexpr int CPR = BK / CE;               // chunks per LDS row
  static constexpr int ROWB = BK * (int)sizeof(T);  // bytes per LDS row
  static constexpr int BYTES = R * ROWB;
  static constexpr int NI = (BYTES + NT * 16 - 1) / (NT * 16);  // loads per thread per stage
  // A tile smaller than one load per thread is loaded by the first BYTES/1024
  // waves only.
  static constexpr bool PARTIAL = BYTES < NT * 16;
  static_assert(PARTIAL ? BYTES % 1024 == 0 : BYTES % (NT * 16) == 0, "tile must be whole wave loads");
  // Loads every thread issues per stage (what a vmcnt wait may count on).
  static constexpr int NI_MIN = PARTIAL ? 0 : NI;
  static_assert(CPR >= 4 && (CPR & (CPR - 1)) == 0, "rows of 4, 8, 16, ... chunks");

  __device__ static __forceinline__ int swz(int row) { return chunk_swizzle(row, CPR); }
  // Byte offset of element (row, col) in the staged tile.
  __device__ static __forceinline__ int elem(int row, int col) {
    return row * ROWB + (((col / CE) ^ swz(row)) * 16) + (col % CE) * (int)sizeof(T);
  }
  // Row and first reduction index of the chunk of load i of thread tid.
  __device__ static __forceinline__ int row_of(int i, int tid = (int)threadIdx.x) {
    return ((i * NT + tid) * 16) / ROWB;
  }
  __device__ static __forceinline__ int kc_of(int i, int tid = (int)threadIdx.x) {
    const int lin = (i * NT + tid) * 16;
    return (((lin % ROWB) / 16) ^ swz(lin / ROWB)) * CE;
  }

  const char* base;  // element (0, 0)
  int64_t ldb;       // row stride in bytes
  int k_valid;
  uint32_t off[NI];  // byte offset of this lane's chunk at k = 0, or kOOB

  // tid: this thread's index (a caller that issues a tile rarely may pass a
  // copy the compiler cannot see through, so that the offsets are computed at
  // the call instead of being kept live across its loops).
  __device__ __forceinline__ void setup(const T* b, int64_t ld, int rows_valid, int kv, int tid = (int)threadIdx.x) {
    ldb = ld * (int64_t)sizeof(T);
    k_valid = kv;
    rebase(b, rows_valid, tid);
  }
  // New rows, same shape.
  __device__ __forceinline__ void rebase(const T* b, int rows_valid, int tid = (int)threadIdx.x) {
    base = reinterpret_cast<const char*>(b);
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int row = row_of(i, tid);
      off[i] = row < rows_valid && row < R ? (uint32_t)(row * ldb + kc_of(i, tid) * (int)sizeof(T)) : kOOB;
    }
  }
  // Stage the reduction slice [k0, k0 + BK) at LDS address lds.  The whole-
  // slice path and the tail path are separate load batches, so the steady
  // state computes no per-lane bounds.
  __device__ __forceinline__ void issue(uint32_t lds, int k0) const {
    const rsrc_t r = make_rsrc(base + (int64_t)k0 * (int)sizeof(T));
    if (PARTIAL && (int)threadIdx.x * 16 >= BYTES) return;  // wave-uniform
    if (k0 + BK <= k_valid) {
      dma_n<NI, NT * 16>(r, off, lds + wave_id() * 1024);
    } else {
      uint32_t v[NI];
#pragma unroll
      for (int i = 0; i < NI; ++i) v[i] = k0 + kc_of(i) >= k_valid ? kOOB : off[i];
      dma_n<NI, NT * 16>(r, v, lds + wave_id() * 1024);
    }
  }
};

template <class T, int R, int BK, int NT = kThreads>
struct RTile {
  typedef RTile Layout;                             // LDS layout (operand reads)
  static constexpr int CE = 16 / (int)sizeof(T);
  static constexpr int ROWB = R * (int)sizeof(T);  // bytes per LDS k-row
  static constexpr int BYTES = BK * ROWB;
  static constexpr int NI = BYTES / (NT * 16);
  static constexpr int NI_MIN = NI;
  static_assert(BYTES % (NT * 16) == 0, "tile must be a whole number of workgroup loads");
  static_assert(ROWB >= 256, "swizzle needs 16 chunks per k-row");

  // The transposing read of a k16 step covers 4 k-rows x 64 bytes per 32
  // lanes; XOR-ing the chunk index by 4 * (k-row % 4) puts those 4 x 64 bytes
  // on all 64 banks.
  __device__ static __forceinline__ int swz(int krow) { return (krow & 3) * 4; }
  __device__ static __forceinline__ int kr_of(int i) { return ((i * NT + (int)threadIdx.x) * 16) / ROWB; }

  const char* base;  // element (r = 0, k = 0)
  int64_t ldb;       // k-row stride in bytes
  int k_valid;
  uint32_t off[NI];

  __device__ __forceinline__ void setup(const T* b, int64_t ld, int rows_valid, int kv) {
    base = reinterpret_cast<const char*>(b);
    ldb = ld * (int64_t)sizeof(T);
    k_valid = kv;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int lin = (i * NT + (int)threadIdx.x) * 16;
      const int kr = lin / ROWB;
      const int r = (((lin % ROWB) / 16) ^ swz(kr)) * CE;
      off[i] = r < rows_valid ? (uint32_t)(kr * ldb + r * (int)sizeof(T)) : kOOB;
    }
  }
  __device__ __forceinline__ void issue(uint32_t lds, int k0) const {
    const rsrc_t rs = make_rsrc(base + (int64_t)k0 * ldb);
    if (k0 + BK <= k_valid) {
      dma_n<NI, NT * 16>(rs, off, lds + wave_id() * 1024);
    } else {
      uint32_t v[NI];
#pragma unroll
      for (int i = 0; i < NI; ++i) v[i] = k0 + kr_of(i) >= k_valid ? kOOB : off[i];
      dma_n<NI, NT * 16>(rs, v, lds + wave_id() * 1024);
    }
  }
};

// MFMA operand (8 reduction values of one row) from a staged tile.  `lane`
// is this lane's index (an epilogue passes an opaque copy, see opaque_zero).
template <class T, int R, int BK, int NT>
__device__ __forceinline__ typename Vec8<T>::type read_op(const KTile<T, R, BK, NT>&, const char* stage, int row,
                                                          int j, int lane = lane_id()) {
  typedef KTile<T, R, BK, NT> KT;
  typedef typename Vec8<T>::type V8;
  const int k = 16 * j + (lane >> 5) * 8;
  const int c = k / KT::CE;
  const char* rowp = stage + row * KT::ROWB;
  if constexpr (sizeof(T) == 2) {
    return *reinterpret_cast<const V8*>(rowp + ((c ^ KT::swz(row)) * 16));
  } else {
    const float4 lo = *reinterpret_cast<const float4*>(rowp + ((c ^ KT::swz(row)) * 16));
    const float4 hi = *reinterpret_cast<const float4*>(rowp + (((c + 1) ^ KT::swz(row)) * 16));
    V8 v;
    v[0] = lo.x; v[1] = lo.y; v[2] = lo.z; v[3] = lo.w;
    v[4] = hi.x; v[5] = hi.y; v[6] = hi.z; v[7] = hi.w;
    return v;
  }
}

template <class T, int R, int BK, int NT>
__device__ __forceinline__ typename Vec8<T>::type read_op(const RTile<T, R, BK, NT>&, const char* stage, int row,
                                                          int j) {
  typedef RTile<T, R, BK, NT> RT;
  typedef typename Vec8<T>::type V8;
  const int lane = lane_id();
  const int kb = 16 * j + (lane >> 5) * 8;
  if constexpr (sizeof(T) == 2) {
    // Transposing read: in each group of 16 lanes, lane 4a+q names row-chunk
    // (k = kb + 4h + a, r = 16*group + 4q) and every lane receives 4 k-values
    // of row (lane % 32).
    const int g = (lane >> 4) & 1, a = (lane & 15) >> 2, q = lane & 3;
    const int r = row - (lane & 31) + 16 * g + 4 * q;  // row is this lane's own row (m0 + lane % 32)
    s16x4_t v[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int krow = kb + 4 * h + a;
      const char* p = stage + krow * RT::ROWB + (((r / RT::CE) ^ RT::swz(krow)) * 16) + (r % RT::CE) * 2;
      v[h] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4_t*)p);
    }
    // the two 4-value halves side by side are the 8 values of the operand
    const s16x8_t both = __builtin_shufflevector(v[0], v[1], 0, 1, 2, 3, 4, 5, 6, 7);
    V8 out;
    __builtin_memcpy(&out, &both, 16);
    return out;
  } else {
    V8 out;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int krow = kb + t;
      out[t] = *reinterpret_cast<const float*>(stage + krow * RT::ROWB + (((row / RT::CE) ^ RT::swz(krow)) * 16) +
                                               (row % RT::CE) * 4);
    }
    return out;
  }
}

// Vocabulary operands packed once per call into the workspace, so every tile
// load is aligned and in bounds: bias as fp32 [V_pad] (-inf past V: padding
// rows drop out of the softmax) and E as [V_pad][DP] in the compute dtype
// (zero past D and V).
template <class T>
__global__ __launch_bounds__(256) void pack_vocab_kernel(const T* __restrict__ E, int64_t lde,
                                                         const float* __restrict__ bias, int V, int D, int V_pad,
                                                         int DP, T* __restrict__ Ep, float* __restrict__ biasp,
                                                         const float* __restrict__ h_scale = nullptr,
                                                         const float* __restrict__ w_scale = nullptr,
                                                         float logit_scale = 0.f, float* __restrict__ multp = nullptr) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e < (int64_t)V_pad * DP) {
    const int v = (int)(e / DP), d = (int)(e % DP);
    Ep[e] = (v < V && d < D) ? E[(int64_t)v * lde + d] : (T)0.f;
  }
  if (e < V_pad) biasp[e] = e < V ? (bias ? bias[e] : 0.f) : kNegInf;
  // e4m3 scores: the factor that turns row v's e4m3 dot product into a score
  if (multp && e < V_pad) multp[e] = e < V ? logit_scale * h_scale[0] * w_scale[e] : 0.f;
}

// Per-lane byte offsets, within one staged slice, of the operands of F
// fragments (rows row0 + 32 f + lane % 32) for the J k16 steps of a slice,
// computed once per reduction so that an operand read is one add of the
// slice base plus the LDS read(s).
//   KTile: one offset per (step, fragment) (the XOR swizzle mixes the step
//          into the chunk index);
//   RTile (2-byte types): one offset per fragment; the step adds 16 k-rows
//          and the second half of the operand 4 k-rows, both immediate
//          offsets of the transposing reads (the swizzle depends only on the
//          k-row modulo 4, which neither changes).
template <class Tile, int F, int J>
struct OpOffsets;

// KTile: the chunk swizzle of a row repeats every 32 rows (chunk_swizzle), so
// fragment f's operand sits 32 f rows (a compile-time byte offset, folded
// into the LDS read's immediate) after fragment 0's: one register per step.
template <class T, int R, int BK, int NT, int F, int J>
struct OpOffsets<KTile<T, R, BK, NT>, F, J> {
  typedef KTile<T, R, BK, NT> KT;
  typedef typename Vec8<T>::type V8;
  static constexpr uint32_t kFragBytes = 32 * KT::ROWB;
  uint32_t off[J];
  __device__ __forceinline__ void init(int row0) {
    const int lane = lane_id();
#pragma unroll
    for (int j = 0; j < J; ++j) off[j] = KT::elem(row0 + (lane & 31), 16 * j + (lane >> 5) * 8);
  }
  __device__ __forceinline__ V8 read(const char* stage, int j, int f) const {
    if constexpr (sizeof(T) == 2) {
      return *reinterpret_cast<const V8*>(stage + off[j] + f * kFragBytes);
    } else {
      // 8 fp32 values span chunks c and c + 1 = c ^ 1 (c even): offsets o and o ^ 16
      // (kFragBytes is a multiple of 32, so the XOR commutes with the fragment offset)
      const float4 lo = *reinterpret_cast<const float4*>(stage + off[j] + f * kFragBytes);
      const float4 hi = *reinterpret_cast<const float4*>(stage + (off[j] ^ 16u) + f * kFragBytes);
      V8 v;
      v[0] = lo.x; v[1] = lo.y; v[2] = lo.z; v[3] = lo.w;
      v[4] = hi.x; v[5] = hi.y; v[6] = hi.z; v[7] = hi.w;
      return v;
    }
  }
};

template <class T, int R, int BK, int NT, int F, int J>
struct OpOffsets<RTile<T, R, BK, NT>, F, J> {
  typedef RTile<T, R, BK, NT> RT;
  typedef typename Vec8<T>::type V8;
  int row0;
  uint32_t off[F];
  __device__ __forceinline__ void init(int r0) {
    row0 = r0;
    if constexpr (sizeof(T) == 2) {
      // lane = 32 hi + 16 g + 4 a + q reads k-row 8 hi + a (+ 16 j + 4 h) at
      // row chunk (row0 + 32 f) / 8 + 2 g + q / 2, XOR 4 a, half q % 2
      const int lane = lane_id();
      const int hi = lane >> 5, g = (lane >> 4) & 1, a = (lane & 15) >> 2, q = lane & 3;
#pragma unroll
      for (int f = 0; f < F; ++f)
        off[f] = (uint32_t)((8 * hi + a) * RT::ROWB + ((((row0 + 32 * f) >> 3) + 2 * g + (q >> 1)) ^ (4 * a)) * 16 +
                            8 * (q & 1));
    }
  }
  __device__ __forceinline__ V8 read(const char* stage, int j, int f) const {
    if constexpr (sizeof(T) == 2) {
      const char* p = stage + off[f] + j * 16 * RT::ROWB;
      const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4_t*)p);
      const s16x4_t hi =
          __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4_t*)(p + 4 * RT::ROWB));
      const s16x8_t both = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      V8 out;
      __builtin_memcpy(&out, &both, 16);
      return out;
    } else {
      return read_op(RT(), stage, row0 + 32 * f + (lane_id() & 31), j);
    }
  }
};

// Block-major transposed tile: the rows of the operand come in groups of 32,
// each group a [BK k-rows][32 rows] sub-tile of its own (the image of one
// 32 x 32 block of a block-tiled source, copied as one contiguous run).  The
// operand reads transpose like RTile's; within a sub-tile a k-row is 64
// bytes (bf16), so the 4 k-rows x 32 bytes that a 16-lane group of a
// transposing read touches fall on 32 distinct banks without any swizzle.
template <class T, int R, int BK, int NT>
struct BRTile {
  typedef BRTile Layout;
  static constexpr int CE = 16 / (int)sizeof(T);
  static constexpr int KROWB = 32 * (int)sizeof(T);  // bytes of one k-row of a sub-tile
  static constexpr int SUB = BK * KROWB;             // bytes of one 32-row sub-tile
  static constexpr int BYTES = R / 32 * SUB;
  static constexpr int NI = BYTES / (NT * 16);
  static constexpr int NI_MIN = NI;
  static_assert(R % 32 == 0 && BYTES % (NT * 16) == 0, "whole sub-tiles, whole workgroup loads");
};

// BRTile: fragment f is sub-tile f after fragment 0's (a compile-time offset).
template <class T, int R, int BK, int NT, int F, int J>
struct OpOffsets<BRTile<T, R, BK, NT>, F, J> {
  typedef BRTile<T, R, BK, NT> BT;
  typedef typename Vec8<T>::type V8;
  uint32_t off0;
  __device__ __forceinline__ void init(int row0) {
    const int lane = lane_id();
    if constexpr (sizeof(T) == 2) {
      // lane = 32 hi + 16 g + 4 a + q reads k-row 8 hi + a (+ 16 j + 4 h) at
      // rows 16 g + 4 q .. + 3 of sub-tile (row0 + 32 f) / 32
      const int hi = lane >> 5, g = (lane >> 4) & 1, a = (lane & 15) >> 2, q = lane & 3;
      off0 = (uint32_t)((row0 >> 5) * BT::SUB + (8 * hi + a) * BT::KROWB + (16 * g + 4 * q) * 2);
    } else {
      // this lane's row (lane % 32) and first k-row (8 (lane / 32))
      off0 = (uint32_t)((row0 >> 5) * BT::SUB + 8 * (lane >> 5) * BT::KROWB + (lane & 31) * 4);
    }
  }
  __device__ __forceinline__ V8 read(const char* stage, int j, int f) const {
    const uint32_t off = off0 + f * BT::SUB;
    if constexpr (sizeof(T) == 2) {
      const char* p = stage + off + j * 16 * BT::KROWB;
      const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4_t*)p);
      const s16x4_t hi =
          __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4_t*)(p + 4 * BT::KROWB));
      const s16x8_t both = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      V8 out;
      __builtin_memcpy(&out, &both, 16);
      return out;
    } else {
      V8 out;
#pragma unroll
      for (int t = 0; t < 8; ++t)
        out[t] = *reinterpret_cast<const float*>(stage + off + (16 * j + t) * BT::KROWB);
      return out;
    }
  }
};

// MFMA operands of one k16 step of a wave's FM x FN grid of 32x32 blocks.
template <class T, int FM, int FN>
struct StepOps {
  typename Vec8<T>::type a[FM], b[FN];
};

// Read the operands of k16 step j of a staged slice.
template <class T, int FM, int FN, class OA, class OB>
__device__ __forceinline__ void load_step(StepOps<T, FM, FN>& o, const OA& ao, const OB& bo, const char* sA,
                                          const char* sB, int j) {
#pragma unroll
  for (int fm = 0; fm < FM; ++fm) o.a[fm] = ao.read(sA, j, fm);
#pragma unroll
  for (int fn = 0; fn < FN; ++fn) o.b[fn] = bo.read(sB, j, fn);
}

template <class T, int FM, int FN>
__device__ __forceinline__ void mma_step(f32x16_t (&acc)[FM][FN], const StepOps<T, FM, FN>& o) {
#pragma unroll
  for (int fm = 0; fm < FM; ++fm)
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) mfma_k16(acc[fm][fn], o.a[fm], o.b[fn]);
}

// The matrix work of one k16 step (operands `cur`) fused with the LDS reads of
// the next step's operands (`nxt`, step j of the slice at sA / sB): the B
// operands are read first; each A operand is read right after the last MFMA
// that uses its predecessor, so only one A operand is double-buffered at a
// time (register budget) while every read still has at least the rest of the
// step's MFMAs to land.
template <class T, int FM, int FN, class OA, class OB>
__device__ __forceinline__ void mma_load_step(f32x16_t (&acc)[FM][FN], const StepOps<T, FM, FN>& cur,
                                              StepOps<T, FM, FN>& nxt, const OA& ao, const OB& bo, const char* sA,
                                              const char* sB, int j) {
#pragma unroll
  for (int fn = 0; fn < FN; ++fn) nxt.b[fn] = bo.read(sB, j, fn);
#pragma unroll
  for (int fm = 0; fm < FM; ++fm) {
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) mfma_k16(acc[fm][fn], cur.a[fm], cur.b[fn]);
    nxt.a[fm] = ao.read(sA, j, fm);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Position of the compute in an NS-deep LDS ring: the slot of the current
// stage and the number of stages after it in the whole walk.
template <int NS>
struct Ring {
  static constexpr int kDepth = NS;
  int slot;
  int remaining;
  // Wait until the next stage has landed and publish it to every wave (which
  // also certifies that every wave has finished reading the stage before it).
  template <int L>
  __device__ __forceinline__ void publish_next() {
    --remaining;
    wait_stages<L, NS>(remaining);
    stage_barrier();
    slot = slot == NS - 1 ? 0 : slot + 1;
  }
};

// acc += A_slice B_slice^T over the nk stages of one output tile, software-
// pipelined: the operands of the next k16 step are read from LDS while the
// current step's matrix work runs, and the wait + barrier that publishes the
// next stage sits between the last two steps of a stage, so neither the LDS
// latency nor the barrier leaves the matrix cores idle at a stage boundary.
// On entry the tile's first stage (ring.slot) is published.  issue_next()
// issues the next pending stage load into the slot that the stage before the
// current one used (free once the current stage is published), or nothing
// when the walk has no more.  On return the ring points at the tile's last
// stage; the caller publishes the next tile's first stage.
template <class T, int BK, int L, int FM, int FN, class TA, class TB, class R, class F>
__device__ __forceinline__ void tile_reduce(f32x16_t (&acc)[FM][FN], const TA& ta, const TB& tb, const char* smem,
                                            int sb, R& ring, int nk, int a_row0, int b_row0, F&& issue_next) {
  constexpr int J = BK / 16;
  OpOffsets<typename TA::Layout, FM, J> ao;
  ao.init(a_row0);
  OpOffsets<typename TB::Layout, FN, J> bo;
  bo.init(b_row0);
  StepOps<T, FM, FN> cur, nxt;
  {
    const char* sA = smem + ring.slot * sb;
    load_step(cur, ao, bo, sA, sA + TA::BYTES, 0);
  }
  // all stages but the last: the next stage is published between the last
  // two k16 steps (the last stage is peeled so no branch splits the MFMAs)
  for (int kt = 0; kt + 1 < nk; ++kt) {
    const char* sA = smem + ring.slot * sb;
    issue_next();
#pragma unroll
    for (int j = 0; j + 1 < J; ++j) {
      mma_load_step(acc, cur, nxt, ao, bo, sA, sA + TA::BYTES, j + 1);
      cur = nxt;
    }
    __builtin_amdgcn_sched_barrier(0);  // the MFMAs above stay ahead of the barrier,
    ring.template publish_next<L>();
    __builtin_amdgcn_sched_barrier(0);  // the ones below stay behind it
    const char* nA = smem + ring.slot * sb;
    mma_load_step(acc, cur, nxt, ao, bo, nA, nA + TA::BYTES, 0);
    cur = nxt;
  }
  {
    const char* sA = smem + ring.slot * sb;
    issue_next();
#pragma unroll
    for (int j = 0; j + 1 < J; ++j) {
      mma_load_step(acc, cur, nxt, ao, bo, sA, sA + TA::BYTES, j + 1);
      cur = nxt;
    }
    mma_step(acc, cur);
  }
}

// tile_reduce over stages that each hold P consecutive slices (slice s of a
// stage at byte s * sb1 of its slot, A then B as in a one-slice stage): one
// wait + barrier per P slices.  nst stages; a stage past the last slice holds
// zeros (its products add nothing).
template <class T, int BK, int P, int L, int FM, int FN, class TA, class TB, class R, class F>
__device__ __forceinline__ void tile_reduce_multi(f32x16_t (&acc)[FM][FN], const TA& ta, const TB& tb,
                                                  const char* smem, int sb, int sb1, R& ring, int nst, int a_row0,
                                                  int b_row0, F&& issue_next) {
  constexpr int J1 = BK / 16, J = P * J1;
  OpOffsets<typename TA::Layout, FM, J1> ao;
  ao.init(a_row0);
  OpOffsets<typename TB::Layout, FN, J1> bo;
  bo.init(b_row0);
  StepOps<T, FM, FN> cur, nxt;
  {
    const char* sA = smem + ring.slot * sb;
    load_step(cur, ao, bo, sA, sA + TA::BYTES, 0);
  }
  for (int kt = 0; kt + 1 < nst; ++kt) {
    const char* st = smem + ring.slot * sb;
    issue_next();
#pragma unroll
    for (int j = 0; j + 1 < J; ++j) {
      const char* sA = st + ((j + 1) / J1) * sb1;
      mma_load_step(acc, cur, nxt, ao, bo, sA, sA + TA::BYTES, (j + 1) % J1);
      cur = nxt;
    }
    __builtin_amdgcn_sched_barrier(0);
    ring.template publish_next<L>();
    __builtin_amdgcn_sched_barrier(0);
    const char* nA = smem + ring.slot * sb;
    mma_load_step(acc, cur, nxt, ao, bo, nA, nA + TA::BYTES, 0);
    cur = nxt;
  }
  {
    const char* st = smem + ring.slot * sb;
    issue_next();
#pragma unroll
    for (int j = 0; j + 1 < J; ++j) {
      const char* sA = st + ((j + 1) / J1) * sb1;
      mma_load_step(acc, cur, nxt, ao, bo, sA, sA + TA::BYTES, (j + 1) % J1);
      cur = nxt;
    }
    mma_step(acc, cur);
  }
}

typedef int i32x8_t __attribute__((ext_vector_type(8)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));

// 32 bytes of e4m3 operand from two 16-byte reads.
__device__ __forceinline__ i32x8_t cat16(bf16x8_t lo, bf16x8_t hi) {
  const i32x4_t l = __builtin_bit_cast(i32x4_t, lo), h = __builtin_bit_cast(i32x4_t, hi);
  return __builtin_shufflevector(l, h, 0, 1, 2, 3, 4, 5, 6, 7);
}

// c += a b over 64 k-values, e4m3 x e4m3 -> fp32 (v_mfma_f32_32x32x64_f8f6f4;
// format code 0 = e4m3 for both operands, no block scales).
__device__ __forceinline__ void mfma_f8_k64(f32x16_t& c, i32x8_t a, i32x8_t b) {
  c = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

// tile_reduce for e4m3 operands packed as if they were bf16 pairs: a staged
// 64-byte row slice holds 64 k-values, and one k64 MFMA consumes it.  Software-
// pipelined like tile_reduce, with the slice as the step.  Each
// lane's 32 operand bytes are the two 16-byte pieces the bf16 reduction reads
// for its two k16 steps (bytes 16 hi .. 16 hi + 15 and 32 + 16 hi .. 32 + 16 hi
// + 15 of the slice, hi = lane / 32).  A and B take the same bytes per lane, so
// whatever order the instruction gives the k-values inside its 64, every
// product pairs h[n, k] with W[v, k] of the same k.
// PIPE = false: one operand set, each slice read and then multiplied (fewer
// registers).
template <int L, bool PIPE, int FM, int FN, class TA, class TB, class R, class F>
__device__ __forceinline__ void tile_reduce_f8(f32x16_t (&acc)[FM][FN], const TA&, const TB&, const char* smem,
                                               int sb, R& ring, int nk, int a_row0, int b_row0, F&& issue_next) {
  OpOffsets<typename TA::Layout, FM, 2> ao;
  ao.init(a_row0);
  OpOffsets<typename TB::Layout, FN, 2> bo;
  bo.init(b_row0);
  auto rd_a = [&](const char* s, int fm) { return cat16(ao.read(s, 0, fm), ao.read(s, 1, fm)); };
  auto rd_b = [&](const char* s, int fn) { return cat16(bo.read(s + TA::BYTES, 0, fn), bo.read(s + TA::BYTES, 1, fn)); };
  if constexpr (!PIPE) {
    for (int kt = 0; kt < nk; ++kt) {
      if (kt > 0) ring.template publish_next<L>();
      const char* sA = smem + ring.slot * sb;
      issue_next();
      i32x8_t b[FN];
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) b[fn] = rd_b(sA, fn);
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        const i32x8_t a = rd_a(sA, fm);
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) mfma_f8_k64(acc[fm][fn], a, b[fn]);
      }
    }
    return;
  }
  // one slice on operands x, with the next slice's operands read into y: the
  // first row of MFMAs goes ahead of the wait + barrier that publishes the next
  // stage, the rest run while y is read
  auto step = [&](const i32x8_t (&xa)[FM], const i32x8_t (&xb)[FN], i32x8_t (&ya)[FM], i32x8_t (&yb)[FN]) {
    issue_next();
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) mfma_f8_k64(acc[0][fn], xa[0], xb[fn]);
    __builtin_amdgcn_sched_barrier(0);
    ring.template publish_next<L>();
    __builtin_amdgcn_sched_barrier(0);
    const char* nA = smem + ring.slot * sb;
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) yb[fn] = rd_b(nA, fn);
    ya[0] = rd_a(nA, 0);
#pragma unroll
    for (int fm = 1; fm < FM; ++fm) {
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) mfma_f8_k64(acc[fm][fn], xa[fm], xb[fn]);
      ya[fm] = rd_a(nA, fm);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  auto last = [&](const i32x8_t (&xa)[FM], const i32x8_t (&xb)[FN]) {
    issue_next();
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) mfma_f8_k64(acc[fm][fn], xa[fm], xb[fn]);
  };
  // two register sets in turn, so no operand is copied between slices
  i32x8_t pa[FM], pb[FN], qa[FM], qb[FN];
  {
    const char* sA = smem + ring.slot * sb;
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) pb[fn] = rd_b(sA, fn);
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) pa[fm] = rd_a(sA, fm);
  }
  int kt = 0;
  for (; kt + 2 < nk; kt += 2) {
    step(pa, pb, qa, qb);
    step(qa, qb, pa, pb);
  }
  if (kt + 1 < nk) {
    step(pa, pb, qa, qb);
    last(qa, qb);
  } else {
    last(pa, pb);
  }
}

// blockIdx -> tile index such that each XCD (blocks are dealt to the 8 XCDs
// round-robin) works through a contiguous range of tile indices, so the tiles
// that run together on one XCD share operands in that XCD's L2.
__device__ __forceinline__ int xcd_swizzle(int b, int n) {
  constexpr int X = 8;
  const int q = n / X;
  if (b >= q * X) return b;
  return (b % X) * q + b / X;
}

// Workgroup index -> (row, col) of an R x Q tile grid such that the 32
// workgroups an XCD runs together cover a G x (32 / G) patch (G rows): blocks
// go to the XCDs round-robin, xcd_swizzle gives each XCD a contiguous range of
// the tile order, and the order walks G-row column strips.
template <int G = 4>
__device__ __forceinline__ void grouped_tile(int b, int R, int Q, int* row, int* col) {
  const int t = xcd_swizzle(b, R * Q);
  const int group = t / (G * Q), first = group * G;
  const int gsize = min(R - first, G);
  *row = first + (t % (G * Q)) % gsize;
  *col = (t % (G * Q)) / gsize;
}

// An LDS ring of NS slots whose stages are not issued at a uniform rate: the
// wait that publishes a stage counts the stages actually issued after it
// (*issued = number of stages issued so far, in stage order; at most 2 of
// them may stay in flight, L loads per thread each).
template <int NS>
struct CountedRing {
  static constexpr int kDepth = NS;
  int slot;            // slot of the current stage
  int cur;             // index of the current stage
  const int* issued;
  template <int L>
  __device__ __forceinline__ void publish_next() {
    ++cur;
    const int ahead = *issued - 1 - cur;
    if (ahead >= 2)
      wait_vmcnt<2 * L>();
    else if (ahead == 1)
      wait_vmcnt<L>();
    else
      wait_vmcnt<0>();
    stage_barrier();
    slot = slot == NS - 1 ? 0 : slot + 1;
  }
};

// ----------------------------------------------------------------------------
// One 16-byte chunk of CE = 16 / sizeof(T) elements in T, read from a source
// of type Src: one 16-byte load when Src is T; two for fp32 rounded to a
// 2-byte T (the cast of autocast with fp32 weights, fused into the packing).
template <class Src, class T>
__device__ __forceinline__ uint4 load_chunk(const Src* p) {
  if constexpr (sizeof(Src) == sizeof(T)) {
    return *reinterpret_cast<const uint4*>(p);
  } else {
    static_assert(sizeof(Src) == 4 && sizeof(T) == 2, "fp32 source, 2-byte dtype");
    const float4 a = *reinterpret_cast<const float4*>(p), b = *reinterpret_cast<const float4*>(p + 4);
    T q[8] = {from_float<T>(a.x), from_float<T>(a.y), from_float<T>(a.z), from_float<T>(a.w),
              from_float<T>(b.x), from_float<T>(b.y), from_float<T>(b.z), from_float<T>(b.w)};
    uint4 u;
    __builtin_memcpy(&u, q, 16);
    return u;
  }
}

// Whether any of the CE values of T in a 16-byte chunk is an infinity or a NaN
// (all exponent bits set).
template <class T>
__device__ __forceinline__ bool chunk_nonfinite(uint4 v) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  bool bad = false;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (sizeof(T) == 4) {
      bad |= (w[i] & 0x7f800000u) == 0x7f800000u;
    } else {
      constexpr uint32_t m = std::is_same<T, f16_t>::value ? 0x7c00u : 0x7f80u;
      bad |= (w[i] & m) == m || ((w[i] >> 16) & m) == m;
    }
  }
  return bad;
}

// Token rows (h) packed in the LDS image of their operand tiles:
// [N_pad / 32][S = K_pad / BK][32 rows][BK], each 16-byte chunk already at its
// XOR-swizzled place (KTile layout), zeros past N and K.  A tile of any
// multiple of 32 rows then loads a reduction slice as contiguous 2 KB runs
// (full cache lines instead of one 64-byte piece per row) with no bounds.
// One workgroup per 32 rows x 8 slices: the rows are read as contiguous
// 512-byte runs into LDS, the 8 slices written as one contiguous 16 KB run.
// The source may be fp32 for a 2-byte T (rounded here); with rowmajor set,
// the rows are also written as a plain [N][K] copy in T.  With rows set, packed
// row q is source row rows[q] for q < n_rows[0] and zero past it (a gather of
// selected tokens in position order).  With nonfinite set, a workgroup that
// packs an infinity or a NaN stores 1 there (every such store writes the same
// value, so the word ends as 1 whatever their order).
// One 32-row x 8-slice tile `grp_s` (32-row group grp_s / SG, slices from (grp_s % SG) * 8)
// of pack_rows_tiled_kernel, by 256 threads (t = 0..255) through `tile` (32 x 33 chunks of
// LDS).  Every thread of the workgroup takes part in the barriers; a caller whose
// threads share a workgroup among several tiles passes grp_s < 0 for threads with no
// tile, which then only keep the barriers.  Returns whether this thread packed a
// non-finite value.
template <class Src, class T>
__device__ __forceinline__ bool pack_rows_tile(int grp_s, int t, uint4* tile, const Src* __restrict__ src, int64_t ld,
                                               int N, int K, int S, T* __restrict__ dst, T* __restrict__ rowmajor,
                                               const int* __restrict__ rows, const int* __restrict__ n_rows) {
  constexpr int BK = SliceK<T>::value, CE = 16 / (int)sizeof(T), CPR = BK / CE;
  static_assert(CPR == 4, "4 chunks per slice row");
  constexpr int SPW = 8;                    // slices per tile
  constexpr int RSTRIDE = SPW * CPR + 1;    // chunks per LDS row (one pad chunk: no bank conflicts)
  const int SG = (S + SPW - 1) / SPW;
  const bool live = grp_s >= 0;
  const int grp = live ? grp_s / SG : 0, s0 = live ? (grp_s % SG) * SPW : 0;
  const int ns = !live ? 0 : S - s0 < SPW ? S - s0 : SPW;
  const int nr = rows ? n_rows[0] : N;
  bool bad = false;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = i * 8 + t / 32, kc = t % 32;
    const int64_t q = (int64_t)grp * 32 + row;
    const int64_t n = q < nr ? (rows ? (int64_t)rows[q] : q) : -1;
    const int k = (s0 * CPR + kc) * CE;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (kc < ns * CPR && n >= 0 && k < K) {
      v = load_chunk<Src, T>(src + n * ld + k);
      if (rowmajor) *reinterpret_cast<uint4*>(rowmajor + n * K + k) = v;
      bad |= chunk_nonfinite<T>(v);
    }
    tile[row * RSTRIDE + kc] = v;
  }
  __syncthreads();
  T* out = dst + ((int64_t)grp * S + s0) * 32 * BK;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int o = i * 256 + t;
    const int sl = o / (32 * CPR), r = (o / CPR) % 32, pc = o % CPR;
    if (sl < ns)
      reinterpret_cast<uint4*>(out)[o] = tile[r * RSTRIDE + sl * CPR + (pc ^ chunk_swizzle(r, CPR))];
  }
  return bad;
}

template <class Src, class T>
__global__ __launch_bounds__(256) void pack_rows_tiled_kernel(const Src* __restrict__ src, int64_t ld, int N, int K,
                                                              int S, T* __restrict__ dst, T* __restrict__ rowmajor,
                                                              const int* __restrict__ rows,
                                                              const int* __restrict__ n_rows,
                                                              int* __restrict__ nonfinite) {
  __shared__ uint4 tile[32 * 33];
  const bool bad = pack_rows_tile<Src, T>((int)blockIdx.x, (int)threadIdx.x, tile, src, ld, N, K, S, dst, rowmajor,
                                          rows, n_rows);
  if (nonfinite && __syncthreads_or(bad) && threadIdx.x == 0) nonfinite[0] = 1;
}

// Pack rows [rows_pad][K] of src (rows_pad a multiple of 32) into the tile image.
// Optional gather and non-finite flag: see pack_rows_tiled_kernel.
struct PackExtra {
  const int* rows = nullptr;
  const int* n_rows = nullptr;
  int* nonfinite = nullptr;
};

template <class T, class Src = T>
__host__ hipError_t launch_pack_rows(const Src* src, int64_t ld, int N, int K, int S, int64_t rows_pad, T* dst,
                                     hipStream_t stream, T* rowmajor = nullptr, PackExtra x = PackExtra()) {
  const int64_t blocks = (rows_pad / 32) * ((S + 7) / 8);
  if (blocks == 0) return hipSuccess;
  pack_rows_tiled_kernel<Src, T><<<(unsigned)blocks, 256, 0, stream>>>(src, ld, N, K, S, dst, rowmajor, x.rows,
                                                                       x.n_rows, x.nonfinite);
  return hipGetLastError();
}

// launch_pack_rows from a source in T, or in fp32 for a 2-byte T.
template <class T>
__host__ hipError_t pack_src(const void* src, int f32, int64_t ld, int rows, int K, int S, int64_t rows_pad, T* dst,
                    hipStream_t stream, T* rowmajor = nullptr, PackExtra x = PackExtra()) {
  if constexpr (sizeof(T) == 2) {
    if (f32)
      return launch_pack_rows<T, float>(static_cast<const float*>(src), ld, rows, K, S, rows_pad, dst, stream,
                                        rowmajor, x);
  }
  return launch_pack_rows<T>(static_cast<const T*>(src), ld, rows, K, S, rows_pad, dst, stream, rowmajor, x);
}

// Loads of a KTile of R token rows (from n0, multiple of 32) from packed rows.
template <class T, int R, int BK, int NT>
struct PackedKLoader {
  typedef KTile<T, R, BK, NT> Layout;
  static constexpr int BYTES = Layout::BYTES, NI = Layout::NI, NI_MIN = Layout::NI_MIN;
  static constexpr bool PARTIAL = Layout::PARTIAL;
  static constexpr int GROUP = 32 * BK * (int)sizeof(T);  // bytes of one 32-row slice
  static_assert(R % 32 == 0 && GROUP % 1024 == 0, "whole 32-row groups, whole wave loads");
  const char* packed;
  const char* base;
  int S;
  uint32_t off[NI];
  __device__ __forceinline__ void setup(const void* pk, int n0, int s_, int tid = (int)threadIdx.x) {
    packed = static_cast<const char*>(pk);
    S = s_;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int lin = i * NT + tid;  // chunk index in the tile image
      off[i] = (uint32_t)((lin / (32 * Layout::CPR)) * S * GROUP + (lin % (32 * Layout::CPR)) * 16);
    }
    rebase(n0);
  }
  __device__ __forceinline__ void rebase(int n0) { base = packed + (int64_t)(n0 >> 5) * S * GROUP; }
  __device__ __forceinline__ void issue(uint32_t lds, int k0) const {
    if (Layout::PARTIAL && (int)threadIdx.x * 16 >= BYTES) return;  // wave-uniform
    const rsrc_t r = make_rsrc(base + (int64_t)(k0 / BK) * GROUP);
    dma_n<NI, NT * 16>(r, off, lds + wave_id() * 1024);
  }
};

// Packed size (elements) and slice count of rows [N_pad][K].
__host__ __device__ __forceinline__ int packed_slices(int64_t K, int bk) {
  const int64_t s = (K + bk - 1) / bk;
  return s > 0 ? (int)s : 1;
}

__device__ __forceinline__ float wave_max32(float x) { return fmaxf(x, __shfl_xor(x, 32)); }
__device__ __forceinline__ float wave_sum32(float x) { return x + __shfl_xor(x, 32); }

}  // namespace swvr
