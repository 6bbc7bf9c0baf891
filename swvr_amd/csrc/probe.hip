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
//      wave tiles), which shows how much the LDS read rate costs;
//   5  as 2 in the hot loops' order: the next step's operands read under the
//      current step's MFMAs (mma_load_step), so no MFMA waits on its own reads;
//   6  the A operands from LDS (4 reads per 8 MFMAs) and the B operands loaded
//      from a 2 MB device array (L2-resident) straight into registers, 8 steps
//      ahead: an operand path that bypasses LDS (iters rounded up to a multiple
//      of 8);
//   7  the hot loops' whole step: mode 5 plus a workgroup barrier every 2 steps
//      and, per 2 steps, 32 KB of direct-to-LDS stage loads (buffer_load ...
//      lds) from the 2 MB array into a 3-slot ring, waited for as the loops
//      wait (the stage traffic every LDS-fed loop here carries; iters rounded
//      up to a multiple of 2);
//   8  as 7 with a barrier every 4 steps and 64 KB of stage loads per 4 steps
//      into a 2-slot ring (two 32-wide slices per stage: half the barriers per
//      MFMA; iters rounded up to a multiple of 4).
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

// Mode 6's register-fed operands: 2 MB of random bf16, filled before the timed launches.
constexpr int kProbeSrc = 1 << 20;  // elements
__device__ bf16_t g_probe_src[kProbeSrc];

__global__ __launch_bounds__(256) void probe_fill_kernel(uint32_t seed) {
  for (int i = blockIdx.x * 256 + threadIdx.x; i < kProbeSrc; i += gridDim.x * 256)
    g_probe_src[i] = random_bf16(mix32(seed ^ (uint32_t)i * 2654435761u));
}

template <int MODE>
__global__ __launch_bounds__(512) void probe_mfma_kernel(int iters, uint32_t seed, float* out) {
  // 32 KB of operands (and, mode 7, a 3-slot ring of 32 KB stages after them)
  __shared__ __attribute__((aligned(1024))) bf16_t lds[16384 + (MODE == 7 ? 3 * 16384 : MODE == 8 ? 4 * 16384 : 0)];
  const int tid = threadIdx.x, lane = lane_id();
  const uint32_t base = mix32(seed ^ (blockIdx.x * 512u + tid));
  for (int i = tid; i < 16384; i += 512) lds[i] = random_bf16(mix32(seed * 31u + i));
  __syncthreads();
  bf16x8_t a[4], b[2];
#pragma unroll
  for (int f = 0; f < 4; ++f)
#pragma unroll
    for (int t = 0; t < 8; ++t) a[f][t] = MODE == 1 ? (bf16_t)0.f : random_bf16(mix32(base + 8 * f + t));
#pragma unroll
  for (int f = 0; f < 2; ++f)
#pragma unroll
    for (int t = 0; t < 8; ++t) b[f][t] = MODE == 1 ? (bf16_t)0.f : random_bf16(mix32(base + 64 + 8 * f + t));
  f32x16_t acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = zero16();
  const char* lb = reinterpret_cast<const char*>(lds);
  const int wb = wave_id() * 1024;
  if constexpr (MODE == 7 || MODE == 8) {
    // stage s (every SPB steps) = NL loads per thread of 16 bytes from the array into slot s % NSL,
    // issued NSL - 1 stages ahead; before the barrier that ends a stage the next one has landed
    constexpr int SPB = MODE == 7 ? 2 : 4, NSL = MODE == 7 ? 3 : 2, NL = 2 * SPB;
    constexpr uint32_t SLOT = NL * 8192u;
    const rsrc_t rs = make_rsrc(g_probe_src);
    const uint32_t ring = lds_addr(lds + 16384);
    auto stage_load = [&](int st) {
      const uint32_t slot = ring + (uint32_t)(st % NSL) * SLOT;
#pragma unroll
      for (int i = 0; i < NL; ++i)
        dma_batch1(rs, ((uint32_t)st * SLOT + (uint32_t)i * 8192u + (uint32_t)threadIdx.x * 16u) &
                           (2u * kProbeSrc - 1u),
                   slot + (uint32_t)i * 8192u + (uint32_t)wave_id() * 1024u);
    };
#pragma unroll
    for (int st = 0; st < NSL - 1; ++st) stage_load(st);
    bf16x8_t na[4], nb[2];
    for (int it = 0; it < iters; it += SPB) {
      stage_load(it / SPB + NSL - 1);
#pragma unroll
      for (int s2 = 0; s2 < SPB; ++s2) {
        const char* win = lb + ((it + s2 + 1) & 3) * 8192 + lane * 16;
#pragma unroll
        for (int f = 0; f < 2; ++f) nb[f] = *reinterpret_cast<const bf16x8_t*>(win + ((wb + (4 + f) * 1024) & 8191));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
          for (int j = 0; j < 2; ++j) mfma_k16(acc[i][j], a[i], b[j]);
          na[i] = *reinterpret_cast<const bf16x8_t*>(win + ((wb + i * 1024) & 8191));
          __builtin_amdgcn_sched_barrier(0);
        }
        if (s2 == SPB - 1) {
          __builtin_amdgcn_sched_barrier(0);
          wait_vmcnt<(NSL - 2) * NL>();  // the next stage has landed; any after it may stay in flight
          stage_barrier();
          __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int f = 0; f < 4; ++f) a[f] = na[f];
#pragma unroll
        for (int f = 0; f < 2; ++f) b[f] = nb[f];
      }
    }
    wait_vmcnt<0>();  // no stage load outstanding when the workgroup ends
  } else if constexpr (MODE == 5) {
    // the hot loops' order: B operands of the next step first, then each A operand after the
    // last MFMA of the current step that uses its predecessor
    bf16x8_t na[4], nb[2];
    for (int it = 0; it < iters; ++it) {
      const char* win = lb + ((it + 1) & 3) * 8192 + lane * 16;
#pragma unroll
      for (int f = 0; f < 2; ++f) nb[f] = *reinterpret_cast<const bf16x8_t*>(win + ((wb + (4 + f) * 1024) & 8191));
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 2; ++j) mfma_k16(acc[i][j], a[i], b[j]);
        na[i] = *reinterpret_cast<const bf16x8_t*>(win + ((wb + i * 1024) & 8191));
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int f = 0; f < 4; ++f) a[f] = na[f];
#pragma unroll
      for (int f = 0; f < 2; ++f) b[f] = nb[f];
    }
  } else if constexpr (MODE == 6) {
    // B from the device array, 8 steps ahead: step s reads 2 KB at (wave base + 2 KB s) mod 2 MB
    constexpr int Q = 8;
    const char* src = reinterpret_cast<const char*>(g_probe_src);
    const uint32_t base = (uint32_t)(blockIdx.x * 8 + wave_id()) * 65536u;
    auto goff = [&](int step, int f) {
      return (base + (uint32_t)step * 2048u + (uint32_t)f * 1024u + (uint32_t)lane * 16u) & (2u * kProbeSrc - 1u);
    };
    bf16x8_t q[Q][2];
#pragma unroll
    for (int s = 0; s < Q; ++s)
#pragma unroll
      for (int f = 0; f < 2; ++f) q[s][f] = *reinterpret_cast<const bf16x8_t*>(src + goff(s, f));
    for (int it = 0; it < iters; it += Q) {
#pragma unroll
      for (int s = 0; s < Q; ++s) {
        const char* win = lb + ((it + s) & 3) * 8192 + lane * 16;
#pragma unroll
        for (int f = 0; f < 4; ++f) a[f] = *reinterpret_cast<const bf16x8_t*>(win + ((wb + f * 1024) & 8191));
        b[0] = q[s][0];
        b[1] = q[s][1];
#pragma unroll
        for (int f = 0; f < 2; ++f) q[s][f] = *reinterpret_cast<const bf16x8_t*>(src + goff(it + s + Q, f));
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j) mfma_k16(acc[i][j], a[i], b[j]);
      }
    }
  }
  for (int it = 0; it < (MODE >= 5 ? 0 : iters); ++it) {
    if constexpr (MODE >= 2) {
      // 16-byte operand reads per step, one 1 KB wave-wide piece each, from the
      // 8 KB window (it % 4) of the 32 KB: offsets stay below 4 * 8192.  MODE 2 reads
      // all six operands (a 128 x 64 wave tile), 3 four (the operand count per MFMA of
      // a 128 x 128 tile), 4 three
      const char* win = lb + (it & 3) * 8192 + lane * 16;
      const int na = MODE == 2 ? 4 : MODE == 3 ? 3 : 2;
#pragma unroll
      for (int f = 0; f < 4; ++f)
        if (f < na) a[f] = *reinterpret_cast<const bf16x8_t*>(win + ((wb + f * 1024) & 8191));
#pragma unroll
      for (int f = 0; f < 2; ++f)
        if (MODE == 2 || f == 0) b[f] = *reinterpret_cast<const bf16x8_t*>(win + ((wb + (4 + f) * 1024) & 8191));
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
  if (mode >= 6) {
    probe_fill_kernel<<<256, 256, 0, stream>>>(0x5eedu);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  timing_begin(kKindProbe, stream);
  switch (mode) {
    case 0: probe_mfma_kernel<0><<<workgroups, 512, 0, stream>>>(iters, 0x5eedu, out); break;
    case 1: probe_mfma_kernel<1><<<workgroups, 512, 0, stream>>>(iters, 0x5eedu, out); break;
    case 2: probe_mfma_kernel<2><<<workgroups, 512, 0, stream>>>(iters, 0x5eedu, out); break;
    case 3: probe_mfma_kernel<3><<<workgroups, 512, 0, stream>>>(iters, 0x5eedu, out); break;
    case 4: probe_mfma_kernel<4><<<workgroups, 512, 0, stream>>>(iters, 0x5eedu, out); break;
    case 5: probe_mfma_kernel<5><<<workgroups, 512, 0, stream>>>(iters, 0x5eedu, out); break;
    case 6: probe_mfma_kernel<6><<<workgroups, 512, 0, stream>>>(iters, 0x5eedu, out); break;
    case 7: probe_mfma_kernel<7><<<workgroups, 512, 0, stream>>>(iters, 0x5eedu, out); break;
    case 8: probe_mfma_kernel<8><<<workgroups, 512, 0, stream>>>(iters, 0x5eedu, out); break;
    default: return hipErrorInvalidValue;
  }
  timing_end(kKindProbe, stream);
  return hipGetLastError();
}

}  // namespace swvr
