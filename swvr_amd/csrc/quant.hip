// OCP e4m3 quantisation of h and W for the e4m3 forward:
//
//   scale = max(amax, 1e-30) * fl(1/448),   q = e4m3(x / scale)  (round to nearest even)
//
// with amax over a row (per-row scales, W) or over the whole matrix (one
// scale, h).  torch divides a tensor by a scalar as a product with the rounded
// reciprocal; computing the scale the same way keeps the bytes identical to a
// quantisation written in torch ops.  One wave per row: the per-row mode finds the row's amax and then
// converts it (the second read of the row hits in L2); the per-tensor mode
// writes the row amaxes, reduces them in one workgroup, and converts with the
// result.  Columns K .. Kp-1 of the output are written as zero bytes.
#include "common.hpp"
#include "launch.hpp"

namespace swvr {

namespace {

constexpr float kE4m3Max = 448.f;
constexpr float kTinyAmax = 1e-30f;

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x = fmaxf(x, __shfl_xor(x, off, 64));
  return x;
}

// Values k .. k+7 of a row (0 past K); vec: 16-byte aligned rows.
template <class Src>
__device__ __forceinline__ void load8(const Src* row, int k, int K, bool vec, float (&v)[8]) {
  if (vec && k + 8 <= K) {
    if constexpr (sizeof(Src) == 2) {
      typedef typename Vec8<Src>::type V8;
      const V8 x = *reinterpret_cast<const V8*>(row + k);
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = (float)x[i];
    } else {
      const float4 a = *reinterpret_cast<const float4*>(row + k);
      const float4 b = *reinterpret_cast<const float4*>(row + k + 4);
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
      v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = k + i < K ? (float)row[k + i] : 0.f;
  }
}

// mode 0: per-row scales (amax, then convert); 1: row amax only; 2: convert
// with scale[0].
template <class Src>
__global__ __launch_bounds__(256) void quant_e4m3_kernel(const Src* __restrict__ x, int64_t ld, int R, int K,
                                                         int Kp, int vec, int mode, float* __restrict__ amax,
                                                         float* __restrict__ scale, uint8_t* __restrict__ out,
                                                         int64_t ldo) {
  const int r = blockIdx.x * 4 + wave_id();
  if (r >= R) return;  // uniform across the wave
  const int lane = lane_id();
  const Src* row = x + (int64_t)r * ld;
  float s;
  if (mode != 2) {
    float m = 0.f;
    for (int k = lane * 8; k < K; k += 512) {
      float v[8];
      load8(row, k, K, vec != 0, v);
#pragma unroll
      for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(v[i]));
    }
    m = wave_max(m);
    if (mode == 1) {
      if (lane == 0) amax[r] = m;
      return;
    }
    s = fmaxf(m, kTinyAmax) * (1.f / kE4m3Max);
    if (lane == 0) scale[r] = s;
  } else {
    s = scale[0];
  }
  uint8_t* orow = out + (int64_t)r * ldo;
  for (int k = lane * 8; k < Kp; k += 512) {
    float v[8];
    load8(row, k, K, vec != 0, v);
    int w0 = __builtin_amdgcn_cvt_pk_fp8_f32(v[0] / s, v[1] / s, 0, false);
    w0 = __builtin_amdgcn_cvt_pk_fp8_f32(v[2] / s, v[3] / s, w0, true);
    int w1 = __builtin_amdgcn_cvt_pk_fp8_f32(v[4] / s, v[5] / s, 0, false);
    w1 = __builtin_amdgcn_cvt_pk_fp8_f32(v[6] / s, v[7] / s, w1, true);
    *reinterpret_cast<int2*>(orow + k) = make_int2(w0, w1);
  }
}

__global__ __launch_bounds__(1024) void amax_reduce_kernel(const float* __restrict__ amax, int R,
                                                           float* __restrict__ scale) {
  __shared__ float sm[16];
  float m = 0.f;
  for (int i = threadIdx.x; i < R; i += 1024) m = fmaxf(m, amax[i]);
  m = wave_max(m);
  if (lane_id() == 0) sm[wave_id()] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.f;
    for (int i = 0; i < 16; ++i) t = fmaxf(t, sm[i]);
    scale[0] = fmaxf(t, kTinyAmax) * (1.f / kE4m3Max);
  }
}

template <class Src>
hipError_t quant_typed(const QuantParams& q, hipStream_t stream) {
  const Src* x = static_cast<const Src*>(q.x);
  const int vec = (reinterpret_cast<uintptr_t>(x) % 16 == 0) && ((q.ld * (int64_t)sizeof(Src)) % 16 == 0);
  const int blocks = (q.R + 3) / 4;
  uint8_t* out = static_cast<uint8_t*>(q.out);
  if (q.per_row) {
    quant_e4m3_kernel<Src><<<blocks, 256, 0, stream>>>(x, q.ld, q.R, q.K, q.Kp, vec, 0, nullptr, q.scale, out, q.ldo);
    return hipGetLastError();
  }
  quant_e4m3_kernel<Src><<<blocks, 256, 0, stream>>>(x, q.ld, q.R, q.K, q.Kp, vec, 1, q.amax, nullptr, nullptr, 0);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  amax_reduce_kernel<<<1, 1024, 0, stream>>>(q.amax, q.R, q.scale);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  quant_e4m3_kernel<Src><<<blocks, 256, 0, stream>>>(x, q.ld, q.R, q.K, q.Kp, vec, 2, nullptr, q.scale, out, q.ldo);
  return hipGetLastError();
}

}  // namespace

hipError_t quant_launch(const QuantParams& q, hipStream_t stream) {
  if (q.R == 0) return hipSuccess;
  timing_begin(kKindQuant, stream);
  hipError_t e;
  switch (q.x_dtype) {
    case kBF16: e = quant_typed<bf16_t>(q, stream); break;
    case kF16: e = quant_typed<f16_t>(q, stream); break;
    default: e = quant_typed<float>(q, stream); break;
  }
  timing_end(kKindQuant, stream);
  return e;
}

}  // namespace swvr
