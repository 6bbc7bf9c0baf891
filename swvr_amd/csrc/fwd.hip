// Fused forward: O = softmax(s * h W^T + b) E and LSE, without writing scores.
//
// Algorithm: the online softmax of swvr/chunked.py:82-105 (docs/DESIGN.md:12-24),
// reorganised for the GPU:
//   * a workgroup owns BM tokens and one of n_split contiguous vocabulary
//     ranges; it walks that range BV rows at a time;
//   * per vocabulary tile it forms S^T = W_tile h_tile^T (BV x BM) with MFMA
//     over the whole hidden size K, double-buffering K slices through LDS;
//   * the 4 waves form a 2 (vocabulary) x 2 (tokens) grid.  In the S^T layout
//     each lane holds one token column, so the softmax max/sum over the
//     vocabulary is a register reduction plus one lane swap;
//   * every wave keeps its own running (m, l, acc) over its half of each tile
//     (an independent partial softmax), and P, rounded to the compute dtype as
//     the reference rounds it (swvr/chunked.py:103, triton_kernels.py:69),
//     feeds acc^T += E^T P^T straight from the score registers;
//   * partials (m, l, acc) of all waves and splits are merged by
//     fwd_combine_kernel in a fixed order (deterministic).
#include "common.hpp"
#include "launch.hpp"

namespace swvr {

namespace {

constexpr int kBK = 32;

// E tile [BV][DP] (row stride DPE) and bias tile [BV], loaded during the
// first stages of the tile's reduction loop.
template <class T, int BV, int DP, int DPE>
struct FwdSide {
  static constexpr int PER = 8;
  static constexpr int TOTAL = BV * DP;
  static constexpr int BATCH = kThreads * PER;
  static constexpr int ITERS = (TOTAL + BATCH - 1) / BATCH;
  T* sE;
  float* sBias;
  const T* E;
  int64_t lde;
  const float* bias;
  int v0, V, D;
  T ev[PER];
  float bv;

  __device__ __forceinline__ void load(int it) {
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int e = (it * PER + q) * kThreads + (int)threadIdx.x;
      const int vv = e / DP, d = e % DP;
      const bool ok = e < TOTAL && v0 + vv < V && d < D;
      ev[q] = ok ? E[(int64_t)(v0 + vv) * lde + d] : (T)0.f;
    }
    if (it == 0 && (int)threadIdx.x < BV) {
      const int v = v0 + (int)threadIdx.x;
      bv = v < V ? (bias ? bias[v] : 0.f) : kNegInf;
    }
  }
  __device__ __forceinline__ void store(int it) {
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int e = (it * PER + q) * kThreads + (int)threadIdx.x;
      if (e < TOTAL) sE[(e / DP) * DPE + e % DP] = ev[q];
    }
    if (it == 0 && (int)threadIdx.x < BV) sBias[threadIdx.x] = bv;
  }
  __device__ __forceinline__ void pre(int kt) {
    if (kt < ITERS) load(kt);
  }
  __device__ __forceinline__ void post(int kt) {
    if (kt < ITERS) store(kt);
  }
  // Batches the reduction loop had no stage for (small K).
  __device__ __forceinline__ void finish(int nk) {
    if (nk < ITERS) {
      for (int it = nk; it < ITERS; ++it) {
        load(it);
        store(it);
      }
      __syncthreads();
    }
  }
};

template <class T, int BV, int BM, int DP>
__global__ __launch_bounds__(kThreads) void fwd_tile_kernel(FwdParams p) {
  typedef typename Vec8<T>::type V8;
  constexpr int LDR = LdsRow<T, kBK>::value;
  constexpr int DPE = DP + 16 / (int)sizeof(T);
  constexpr int FV = BV / 64, FT = BM / 64;  // 32x32 blocks per wave (2x2 waves)
  constexpr int DB = DP / 32;

  __shared__ __attribute__((aligned(16))) T sW[2][BV * LDR];
  __shared__ __attribute__((aligned(16))) T sH[2][BM * LDR];
  __shared__ __attribute__((aligned(16))) T sE[BV * DPE];
  __shared__ float sBias[BV];

  const int lane = lane_id(), w = wave_id();
  const int wv = w >> 1, wt = w & 1;
  const int t = xcd_swizzle(blockIdx.x, p.n_tb * p.n_split);
  const int split = t / p.n_tb, tb = t % p.n_tb;
  const int n0 = tb * BM;
  const int vt_begin = (int)((int64_t)split * p.n_vt / p.n_split);
  const int vt_end = (int)((int64_t)(split + 1) * p.n_vt / p.n_split);
  const T* h = static_cast<const T*>(p.h);
  const T* W = static_cast<const T*>(p.W);

  float m[FT], l[FT];
  f32x16_t oacc[DB][FT];
#pragma unroll
  for (int ft = 0; ft < FT; ++ft) {
    m[ft] = kNegInf;
    l[ft] = 0.f;
#pragma unroll
    for (int db = 0; db < DB; ++db) oacc[db][ft] = zero16();
  }

  KTile<T, BV, kBK> ta;
  ta.ld = p.ldw;
  ta.k_valid = p.K;
  KTile<T, BM, kBK> tbh;
  tbh.base = h + (int64_t)n0 * p.ldh;
  tbh.ld = p.ldh;
  tbh.rows_valid = p.N - n0;
  tbh.k_valid = p.K;
  const int nk = (p.K + kBK - 1) / kBK;

  for (int vt = vt_begin; vt < vt_end; ++vt) {
    const int v0 = vt * BV;
    ta.base = W + (int64_t)v0 * p.ldw;
    ta.rows_valid = p.V - v0;
    FwdSide<T, BV, DP, DPE> side;
    side.sE = sE;
    side.sBias = sBias;
    side.E = static_cast<const T*>(p.E);
    side.lde = p.lde;
    side.bias = p.bias;
    side.v0 = v0;
    side.V = p.V;
    side.D = p.D;

    f32x16_t sacc[FV][FT];
#pragma unroll
    for (int fv = 0; fv < FV; ++fv)
#pragma unroll
      for (int ft = 0; ft < FT; ++ft) sacc[fv][ft] = zero16();

    reduce_loop<T, kBK, FV, FT>(sacc, ta, tbh, sW[0], sW[1], sH[0], sH[1], p.K, wv * (BV / 2), wt * (BM / 2),
                                side);
    side.finish(nk);

    // ---- scores -> running softmax of this wave's half tile
    float mx[FT];
#pragma unroll
    for (int ft = 0; ft < FT; ++ft) mx[ft] = kNegInf;
#pragma unroll
    for (int fv = 0; fv < FV; ++fv)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float b = sBias[wv * (BV / 2) + fv * 32 + c_row(r, lane)];
#pragma unroll
        for (int ft = 0; ft < FT; ++ft) {
          const float x = sacc[fv][ft][r] * p.scale + b;
          sacc[fv][ft][r] = x;
          mx[ft] = fmaxf(mx[ft], x);
        }
      }
#pragma unroll
    for (int ft = 0; ft < FT; ++ft) {
      const float mnew = fmaxf(m[ft], wave_max32(mx[ft]));
      // a column whose scores so far are all -inf keeps m = -inf; shift it by 0
      // (swvr/chunked.py:98-99)
      const float shift = mnew == kNegInf ? 0.f : mnew;
      const float alpha = fast_exp(m[ft] - shift);
      m[ft] = mnew;
      float rs = 0.f;
#pragma unroll
      for (int fv = 0; fv < FV; ++fv)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float pv = fast_exp(sacc[fv][ft][r] - shift);
          sacc[fv][ft][r] = pv;
          rs += pv;
        }
      l[ft] = l[ft] * alpha + wave_sum32(rs);
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[db][ft][r] *= alpha;
    }

    // ---- acc^T[d][token] += E^T[d][v] P^T[v][token]
    // Score registers 8c..8c+7 of a block are the B operand of one k16 step;
    // they hold vocabulary rows 16c + 8(t/4) + 4(lane/32) + t%4, t = 0..7, so
    // the E^T operand is gathered from LDS with the same row order.
#pragma unroll
    for (int fv = 0; fv < FV; ++fv)
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        V8 av[DB];
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
          for (int tt = 0; tt < 8; ++tt) {
            const int vv = wv * (BV / 2) + fv * 32 + 16 * c + 8 * (tt >> 2) + (lane >> 5) * 4 + (tt & 3);
            av[db][tt] = sE[vv * DPE + db * 32 + (lane & 31)];
          }
#pragma unroll
        for (int ft = 0; ft < FT; ++ft) {
          V8 bv;
#pragma unroll
          for (int tt = 0; tt < 8; ++tt) bv[tt] = from_float<T>(sacc[fv][ft][8 * c + tt]);
#pragma unroll
          for (int db = 0; db < DB; ++db) mfma_k16(oacc[db][ft], av[db], bv);
        }
      }
  }

  // ---- partial (m, l, acc) of this wave's vocabulary half of this split
  const int part = split * 2 + wv;
#pragma unroll
  for (int ft = 0; ft < FT; ++ft) {
    const int n = n0 + wt * (BM / 2) + ft * 32 + (lane & 31);
    if (n < p.N) {
      if (lane < 32) {
        p.part_m[(int64_t)part * p.N + n] = m[ft];
        p.part_l[(int64_t)part * p.N + n] = l[ft];
      }
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int d = db * 32 + c_row(r, lane);
          p.part_acc[((int64_t)part * DP + d) * p.N + n] = oacc[db][ft][r];
        }
    }
  }
}

// Merge the partial softmaxes in a fixed order: O = sum_p acc_p e^(m_p - M) /
// sum_p l_p e^(m_p - M), LSE = M + log(...).  A row with every score -inf ends
// with M = -inf, L = 0: O = NaN and LSE = -inf, as swvr/chunked.py:105 gives.
__global__ __launch_bounds__(256) void fwd_combine_kernel(const float* __restrict__ part_m,
                                                          const float* __restrict__ part_l,
                                                          const float* __restrict__ part_acc, int n_part, int N,
                                                          int D, int DP, float* __restrict__ O,
                                                          float* __restrict__ lse) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  float M = kNegInf;
  for (int q = 0; q < n_part; ++q) M = fmaxf(M, part_m[(int64_t)q * N + n]);
  const float shift = M == kNegInf ? 0.f : M;
  float L = 0.f;
  for (int q = 0; q < n_part; ++q) L += part_l[(int64_t)q * N + n] * expf(part_m[(int64_t)q * N + n] - shift);
  for (int d = 0; d < D; ++d) {
    float a = 0.f;
    for (int q = 0; q < n_part; ++q)
      a += part_acc[((int64_t)q * DP + d) * N + n] * expf(part_m[(int64_t)q * N + n] - shift);
    O[(int64_t)n * D + d] = a / L;
  }
  lse[n] = M + logf(L);
}

template <class T, int BV, int BM, int DP>
hipError_t launch_tile(const FwdPlan& plan, const FwdParams& p, hipStream_t stream) {
  const int blocks = plan.n_tb * plan.n_split;
  timing_begin(kKindFwdTile, stream);
  fwd_tile_kernel<T, BV, BM, DP><<<blocks, kThreads, 0, stream>>>(p);
  timing_end(kKindFwdTile, stream);
  return hipGetLastError();
}

// Tile shape per (dtype, padded D): the per-wave score block and the acc^T
// block share the register file, and E plus two K-slices of W and h share LDS.
template <class T, int DP>
struct FwdTile {
  static constexpr bool wide = sizeof(T) == 2;
  static constexpr int BV = wide ? (DP <= 128 ? 256 : 128) : 128;
  static constexpr int BM = wide ? 128 : (DP <= 64 ? 128 : 64);
};

template <class T, int DP>
hipError_t dispatch_tile(const FwdPlan& plan, const FwdParams& p, hipStream_t stream) {
  typedef FwdTile<T, DP> C;
  if (plan.BV != C::BV || plan.BM != C::BM) return hipErrorInvalidValue;
  return launch_tile<T, C::BV, C::BM, DP>(plan, p, stream);
}

template <class T>
hipError_t dispatch_dp(const FwdPlan& plan, const FwdParams& p, hipStream_t stream) {
  switch (plan.DP) {
    case 32: return dispatch_tile<T, 32>(plan, p, stream);
    case 64: return dispatch_tile<T, 64>(plan, p, stream);
    case 128: return dispatch_tile<T, 128>(plan, p, stream);
    case 256:
      if constexpr (sizeof(T) == 2) return dispatch_tile<T, 256>(plan, p, stream);
      return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
}

template <class T>
void tile_of(int DP, int* BV, int* BM) {
  switch (DP) {
    case 32: *BV = FwdTile<T, 32>::BV; *BM = FwdTile<T, 32>::BM; break;
    case 64: *BV = FwdTile<T, 64>::BV; *BM = FwdTile<T, 64>::BM; break;
    case 128: *BV = FwdTile<T, 128>::BV; *BM = FwdTile<T, 128>::BM; break;
    default: *BV = FwdTile<T, 256>::BV; *BM = FwdTile<T, 256>::BM; break;
  }
}

}  // namespace

bool fwd_plan(int dtype, int64_t N, int64_t K, int64_t V, int64_t D, FwdPlan* plan) {
  (void)K;
  const int DP = D <= 32 ? 32 : D <= 64 ? 64 : D <= 128 ? 128 : D <= 256 ? 256 : 0;
  if (DP == 0) return false;
  int BV, BM;
  if (dtype == kF32) {
    if (DP > 128) return false;
    tile_of<float>(DP, &BV, &BM);
  } else if (dtype == kBF16 || dtype == kF16) {
    tile_of<bf16_t>(DP, &BV, &BM);
  } else {
    return false;
  }
  plan->BV = BV;
  plan->BM = BM;
  plan->DP = DP;
  plan->n_tb = (int)((N + BM - 1) / BM);
  plan->n_vt = (int)((V + BV - 1) / BV);
  // Enough workgroups to fill 256 CUs several times over, at least two
  // vocabulary tiles per split.
  int n_split = 1;
  if (plan->n_tb > 0) {
    const int target = 2048;
    n_split = (target + plan->n_tb - 1) / plan->n_tb;
    const int max_split = plan->n_vt / 2 > 1 ? plan->n_vt / 2 : 1;
    if (n_split > max_split) n_split = max_split;
    if (n_split < 1) n_split = 1;
  }
  plan->n_split = n_split;
  plan->n_part = 2 * n_split;
  const size_t per = (size_t)N * sizeof(float);
  plan->ws_bytes = (size_t)plan->n_part * per * (2 + (size_t)DP) + 256;
  return true;
}

hipError_t fwd_launch(int dtype, const FwdPlan& plan, FwdParams p, float* O, float* lse, hipStream_t stream) {
  if (p.N == 0) return hipSuccess;
  p.n_tb = plan.n_tb;
  p.n_split = plan.n_split;
  p.n_vt = plan.n_vt;
  hipError_t e;
  switch (dtype) {
    case kBF16: e = dispatch_dp<bf16_t>(plan, p, stream); break;
    case kF16: e = dispatch_dp<f16_t>(plan, p, stream); break;
    case kF32: e = dispatch_dp<float>(plan, p, stream); break;
    default: return hipErrorInvalidValue;
  }
  if (e != hipSuccess) return e;
  timing_begin(kKindFwdCombine, stream);
  fwd_combine_kernel<<<(p.N + 255) / 256, 256, 0, stream>>>(p.part_m, p.part_l, p.part_acc, plan.n_part, p.N, p.D,
                                                             plan.DP, O, lse);
  timing_end(kKindFwdCombine, stream);
  return hipGetLastError();
}

}  // namespace swvr
