// Matrix-core throughput probe (measurement only; no part of the readout).
//
// Each wave runs `iters` rounds of the hot loops' k16 step shape: a 4 x 2
// grid of 32x32x16 bf16 MFMAs (a 128 x 64 wave tile, eight independent
// accumulator chains), with no memory traffic besides the operand source
// chosen by `mode`:
//   0  random bf16 operands held in registers (values spread like N(0,1) data);
//   1  zero operands in registers (the same instructions at the lowest power);
//   2  random operands read from LDS every step, 6 x 16-byte reads per 8
//      MFMAs, as the forward / gradient GEMM loops read them;
//   3, 4  the same with 4 and 3 reads per 8 MFMAs (the read rate of larger
//      wave tiles), which shows how much the LDS read rate costs.
// Comparing the rates shows how much of the datasheet peak this chip reaches
// with the operand data and LDS traffic of the real kernels, i.e. the ceiling
// that power and clock set for them.
#include "common.hpp"
#include "launch.hpp"

namespace swvr {

namespace {

__device__ __forceinline__ uint32_t mix32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352dU;
  x ^= x >> 15;
  x *= 0x846ca68bU;
  x ^= x >> 16;
  return x;
}

// A bf16 value of magnitude 2^-2 .. 2^2 with random sign and mantissa.
__device__ __forceinline__ bf16_t random_bf16(uint32_t h) {
  const uint32_t sign = (h & 1u) << 15, exp = 125u + ((h >> 1) & 3u), man = (h >> 3) & 0x7fu;
  const uint16_t bits = (uint16_t)(sign | (exp << 7) | man);
  bf16_t v;
  __builtin_memcpy(&v, &bits, 2);
  return v;
}

__global__ __launch_bounds__(512) void probe_mfma_kernel(int iters, int mode, uint32_t seed, float* out) {
  __shared__ __attribute__((aligned(1024))) bf16_t lds[16384];  // 32 KB of operands
  const int tid = threadIdx.x, lane = lane_id();
  const uint32_t base = mix32(seed ^ (blockIdx.x * 512u + tid));
  for (int i = tid; i < 16384; i += 512) lds[i] = random_bf16(mix32(seed * 31u + i));
  __syncthreads();
  bf16x8_t a[4], b[2];
#pragma unroll
  for (int f = 0; f < 4; ++f)
#pragma unroll
    for (int t = 0; t < 8; ++t) a[f][t] = mode == 1 ? (bf16_t)0.f : random_bf16(mix32(base + 8 * f + t));
#pragma unroll
  for (int f = 0; f < 2; ++f)
#pragma unroll
    for (int t = 0; t < 8; ++t) b[f][t] = mode == 1 ? (bf16_t)0.f : random_bf16(mix32(base + 64 + 8 * f + t));
  f32x16_t acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = zero16();
  const char* lb = reinterpret_cast<const char*>(lds);
  const int wb = wave_id() * 1024;
  for (int it = 0; it < iters; ++it) {
    if (mode >= 2) {
      // 16-byte operand reads per step, one 1 KB wave-wide piece each, from the
      // 8 KB window (it % 4) of the 32 KB: offsets stay below 4 * 8192.  mode 2 reads
      // all six operands (a 128 x 64 wave tile), 3 four (the operand count per MFMA of
      // a 128 x 128 tile), 4 three
      const char* win = lb + (it & 3) * 8192 + lane * 16;
      const int na = mode == 2 ? 4 : mode == 3 ? 3 : 2;
#pragma unroll
      for (int f = 0; f < 4; ++f)
        if (f < na) a[f] = *reinterpret_cast<const bf16x8_t*>(win + ((wb + f * 1024) & 8191));
#pragma unroll
      for (int f = 0; f < 2; ++f)
        if (mode == 2 || f == 0) b[f] = *reinterpret_cast<const bf16x8_t*>(win + ((wb + (4 + f) * 1024) & 8191));
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) mfma_k16(acc[i][j], a[i], b[j]);
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) s += acc[i][j][r];
  out[(int64_t)blockIdx.x * 512 + tid] = s;
}

}  // namespace

hipError_t probe_mfma(int workgroups, int iters, int mode, float* out, hipStream_t stream) {
  timing_begin(kKindProbe, stream);
  probe_mfma_kernel<<<workgroups, 512, 0, stream>>>(iters, mode, 0x5eedu, out);
  timing_end(kKindProbe, stream);
  return hipGetLastError();
}

}  // namespace swvr
