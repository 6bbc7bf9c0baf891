// MSE readout loss over the forward's outputs (swvr/api.py:53-66):
//
//   per_tok[n] = w[n] * ( mean_d (O[n,d] - target[n,d])^2 + z * lse[n]^2 )
//   loss       = sum_n per_tok[n] * c,   c = 1 / sum_n w[n]  (mean, weighted)
//                                          1 / N            (mean, unweighted)
//                                          1                (sum)
//
// and the loss's derivatives up to the scalar c (which the host multiplies in
// together with the incoming gradient):
//
//   gO[n,d] = w[n] * (2 / D) * (O[n,d] - target[n,d]),   glse[n] = w[n] * 2 z lse[n].
//
// mse_token_kernel: one wave per token (lanes over d), 16 tokens per
// workgroup; writes per_tok (reduction "none"), gO, glse, and the
// workgroup's sums of per_tok and w in token order.  mse_reduce_kernel: one
// workgroup adds the partial sums in a fixed order, so the loss is the same
// on every run.
#include <mutex>

#include "common.hpp"
#include "launch.hpp"

namespace swvr {

namespace {

constexpr int kLossTokensPerWave = 4;
constexpr int kLossTokensPerBlock = 4 * kLossTokensPerWave;

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}

template <class TT>
__global__ __launch_bounds__(256) void mse_token_kernel(const float* __restrict__ O, const float* __restrict__ lse,
                                                        const TT* __restrict__ target, int64_t ldt,
                                                        const float* __restrict__ weight, int N, int D, float z,
                                                        float* __restrict__ per_tok, float* __restrict__ gO,
                                                        float* __restrict__ glse, float* __restrict__ part,
                                                        int n_blk) {
  __shared__ float s_loss[4], s_w[4];
  const int lane = lane_id(), wv = wave_id();
  const float inv_d = 1.f / (float)D, two_d = 2.f / (float)D;
  float wave_loss = 0.f, wave_w = 0.f;
  for (int j = 0; j < kLossTokensPerWave; ++j) {
    const int n = blockIdx.x * kLossTokensPerBlock + wv * kLossTokensPerWave + j;
    if (n >= N) break;  // uniform across the wave
    const float w = weight ? weight[n] : 1.f;
    const float* o = O + (int64_t)n * D;
    const TT* t = target + (int64_t)n * ldt;
    float sq = 0.f;
    for (int d = lane; d < D; d += 64) {
      const float diff = o[d] - to_float(t[d]);
      sq += diff * diff;
      if (gO) gO[(int64_t)n * D + d] = w * two_d * diff;
    }
    sq = wave_sum(sq);
    const float l = lse[n];
    float tok = sq * inv_d;
    if (z != 0.f) tok += z * (l * l);
    tok *= w;
    if (lane == 0) {
      if (per_tok) per_tok[n] = tok;
      if (glse) glse[n] = z != 0.f ? w * (2.f * z) * l : 0.f;
    }
    wave_loss += tok;
    wave_w += w;
  }
  if (lane == 0) {
    s_loss[wv] = wave_loss;
    s_w[wv] = wave_w;
  }
  __syncthreads();
  if (threadIdx.x == 0 && part) {
    part[blockIdx.x] = ((s_loss[0] + s_loss[1]) + s_loss[2]) + s_loss[3];
    part[n_blk + blockIdx.x] = ((s_w[0] + s_w[1]) + s_w[2]) + s_w[3];
  }
}

// mode: SWVR_REDUCE_SUM or SWVR_REDUCE_MEAN; weighted: the mean divides by sum w.
__global__ __launch_bounds__(256) void mse_reduce_kernel(const float* __restrict__ part, int n_blk, int N,
                                                         int mean, int weighted, float* __restrict__ out,
                                                         float* __restrict__ scale) {
  __shared__ float s_loss[256], s_w[256];
  float a = 0.f, b = 0.f;
  for (int i = threadIdx.x; i < n_blk; i += 256) {
    a += part[i];
    b += part[n_blk + i];
  }
  s_loss[threadIdx.x] = a;
  s_w[threadIdx.x] = b;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) {
      s_loss[threadIdx.x] += s_loss[threadIdx.x + s];
      s_w[threadIdx.x] += s_w[threadIdx.x + s];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const float total = s_loss[0];
    if (!mean) {
      out[0] = total;
      if (scale) scale[0] = 1.f;
    } else {
      const float denom = weighted ? s_w[0] : (float)N;
      out[0] = total / denom;
      if (scale) scale[0] = 1.f / denom;
    }
  }
}

template <class TT>
hipError_t launch_token(const MseParams& p, int n_blk, float* part, hipStream_t stream) {
  mse_token_kernel<TT><<<n_blk, 256, 0, stream>>>(p.O, p.lse, static_cast<const TT*>(p.target), p.ldt, p.weight,
                                                  p.N, p.D, p.z, p.per_tok, p.gO, p.glse, part, n_blk);
  return hipGetLastError();
}

// Scratch of the allocation-free entry point (swvr_mse_loss_noalloc): the
// per-workgroup partial sums of up to kMseNoAllocMaxTokens tokens.  Each device
// holds its own copy for the life of the process; its address comes from
// hipGetSymbolAddress (the name itself is a host-side stand-in in host code).
constexpr int kNoAllocMaxBlocks = (kMseNoAllocMaxTokens + kLossTokensPerBlock - 1) / kLossTokensPerBlock;
static __device__ __align__(256) float scratch[2 * kNoAllocMaxBlocks];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

}  // namespace

hipError_t mse_noalloc_scratch(hipStream_t stream, void** ptr) {
  // the device the kernels will run on: the stream's (the null stream: the current device's)
  int dev = -1;
  hipError_t e = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    // the array's address on that device, looked up with it current
    int cur = -1;
    e = hipGetDevice(&cur);
    if (e != hipSuccess) return e;
    if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return e;
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev) {
      const hipError_t r = hipSetDevice(cur);
      if (e == hipSuccess) e = r;
    }
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return hipSuccess;
}

size_t mse_workspace_bytes(int N) {
  const int64_t n_blk = ((int64_t)N + kLossTokensPerBlock - 1) / kLossTokensPerBlock;
  return (size_t)(2 * n_blk) * sizeof(float);
}

hipError_t mse_launch(const MseParams& p, void* ws, hipStream_t stream) {
  const int n_blk = (p.N + kLossTokensPerBlock - 1) / kLossTokensPerBlock;
  float* part = p.reduce ? static_cast<float*>(ws) : nullptr;
  hipError_t e = hipSuccess;
  timing_begin(kKindLoss, stream);
  if (n_blk > 0) {
    switch (p.target_dtype) {
      case 0: e = launch_token<bf16_t>(p, n_blk, part, stream); break;
      case 1: e = launch_token<f16_t>(p, n_blk, part, stream); break;
      default: e = launch_token<float>(p, n_blk, part, stream); break;
    }
  }
  if (e == hipSuccess && p.reduce) {
    mse_reduce_kernel<<<1, 256, 0, stream>>>(part, n_blk, p.N, p.reduce == 2, p.weight != nullptr, p.out,
                                             p.scale);
    e = hipGetLastError();
  }
  timing_end(kKindLoss, stream);
  return e;
}

}  // namespace swvr
