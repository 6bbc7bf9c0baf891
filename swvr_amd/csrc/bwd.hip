// Backward of the readout (docs/DESIGN.md:26-37, swvr/chunked.py:108-151).
//
//   delta = rowsum(O * gO) - gLSE                                 bwd_delta_kernel
//   per vocabulary chunk [v0, v0 + C):
//     P  = exp(s * h W_c^T + b_c - LSE)        (scores recomputed)
//     dS = P * (gO E_c^T - delta)                                 bwd_scores_kernel
//       -> stage s*dS in the compute dtype (what the gradient GEMMs consume,
//          swvr/chunked.py:143-145 / triton_kernels.py:108-109)
//       -> dE_c = P^T gO and db_c = colsum(dS), accumulated per token group
//          in registers and written as partials (no atomics)
//     dW_c = stage^T h   and   dh += stage W_c                    bwd_gemm_kernel
//     dE_c, db_c = fixed-order sum of the partials                bwd_reduce_kernel
// Every reduction has a fixed order, so gradients are bitwise reproducible.
#include "common.hpp"
#include "launch.hpp"

namespace swvr {

namespace {

constexpr int kBK = 32;

__device__ __forceinline__ void store_as(void* base, int64_t idx, int dtype, float v) {
  if (dtype == kBF16)
    static_cast<bf16_t*>(base)[idx] = (bf16_t)v;
  else if (dtype == kF16)
    static_cast<f16_t*>(base)[idx] = (f16_t)v;
  else
    static_cast<float*>(base)[idx] = v;
}

// ---------------------------------------------------------------- delta
__global__ __launch_bounds__(256) void bwd_delta_kernel(const float* __restrict__ O, const float* __restrict__ gO,
                                                        const float* __restrict__ glse, int N, int D,
                                                        float* __restrict__ delta) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  float s = 0.f;
  for (int d = 0; d < D; ++d) s += O[(int64_t)n * D + d] * gO[(int64_t)n * D + d];
  delta[n] = s - glse[n];
}

// ---------------------------------------------------------------- scores
struct ScoresParams {
  const void* h;
  int64_t ldh;
  const void* W;
  int64_t ldw;
  const void* E;
  int64_t lde;
  const float* bias;
  float scale;
  int N, K, D;
  const float* lse;
  const float* delta;
  const float* gO;  // fp32 [N][D]
  int v0, cv;       // chunk start and rows
  int C;            // chunk stride of the partials (multiple of BV)
  int n_tb, G, n_vtc;
  void* stage;      // [C][ld_stage] compute dtype, token index contiguous
  int64_t ld_stage;
  float* part_dE;   // [G][DP][C]
  float* part_db;   // [G][C]
  int need_stage, need_dE, need_db;
};

// gO tile (rounded to the compute dtype, as swvr/chunked.py:115 rounds it),
// LSE and delta of one token block, loaded during the first stages of the
// block's reduction loop.
template <class T, int BM, int DP, int DPE>
struct ScoresSide {
  static constexpr int PER = 8;
  static constexpr int TOTAL = BM * DP;
  static constexpr int BATCH = kThreads * PER;
  static constexpr int ITERS = (TOTAL + BATCH - 1) / BATCH;
  T* sG;
  float* sLse;
  float* sDelta;
  const float* gO;
  const float* lse;
  const float* delta;
  int n0, N, D;
  float gv[PER];
  float lv, dv;

  __device__ __forceinline__ void load(int it) {
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int e = (it * PER + q) * kThreads + (int)threadIdx.x;
      const int tl = e / DP, d = e % DP;
      const bool ok = e < TOTAL && n0 + tl < N && d < D;
      gv[q] = ok ? gO[(int64_t)(n0 + tl) * D + d] : 0.f;
    }
    if (it == 0 && (int)threadIdx.x < BM) {
      const int n = n0 + (int)threadIdx.x;
      // padding tokens: P = exp(x - inf) = 0
      lv = n < N ? lse[n] : kPosInf;
      dv = n < N ? delta[n] : 0.f;
    }
  }
  __device__ __forceinline__ void store(int it) {
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int e = (it * PER + q) * kThreads + (int)threadIdx.x;
      if (e < TOTAL) sG[(e / DP) * DPE + e % DP] = from_float<T>(gv[q]);
    }
    if (it == 0 && (int)threadIdx.x < BM) {
      sLse[threadIdx.x] = lv;
      sDelta[threadIdx.x] = dv;
    }
  }
  __device__ __forceinline__ void pre(int kt) {
    if (kt < ITERS) load(kt);
  }
  __device__ __forceinline__ void post(int kt) {
    if (kt < ITERS) store(kt);
  }
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

// One workgroup: BV vocabulary rows of the chunk x one group of token
// blocks.  Waves split the BV rows four ways, so dE / db of a vocabulary row
// live in one wave's registers for the whole group.  Scores use the S layout
// (A = h rows, B = W rows): a lane holds one vocabulary column and the
// registers hold tokens, which is the B-operand layout P needs for
// dE^T = gO^T P.
template <class T, int BM, int BV, int DP>
__global__ __launch_bounds__(kThreads) void bwd_scores_kernel(ScoresParams p) {
  typedef typename Vec8<T>::type V8;
  constexpr int LDR = LdsRow<T, kBK>::value;
  constexpr int DPE = DP + 16 / (int)sizeof(T);
  constexpr int FT = BM / 32, FV = BV / 128;
  constexpr int DB = DP / 32, DK = DP / 16;
  constexpr int WVR = BV / 4;  // vocabulary rows per wave

  __shared__ __attribute__((aligned(16))) T sH[2][BM * LDR];
  __shared__ __attribute__((aligned(16))) T sW[2][BV * LDR];
  __shared__ __attribute__((aligned(16))) T sE[BV * DPE];
  __shared__ __attribute__((aligned(16))) T sG[BM * DPE];
  __shared__ float sBias[BV];
  __shared__ float sLse[BM];
  __shared__ float sDelta[BM];

  const int lane = lane_id(), w = wave_id();
  const int t = xcd_swizzle(blockIdx.x, p.n_vtc * p.G);
  const int vt = t / p.G, g = t % p.G;
  const int vl0 = vt * BV;      // first chunk-local row of this tile
  const int vg0 = p.v0 + vl0;   // its global row
  const int rows = p.cv - vl0;  // valid rows of this tile (may exceed BV)
  const int tb_begin = (int)((int64_t)g * p.n_tb / p.G);
  const int tb_end = (int)((int64_t)(g + 1) * p.n_tb / p.G);
  const T* E = static_cast<const T*>(p.E);

  for (int e = threadIdx.x; e < BV * DP; e += kThreads) {
    const int vv = e / DP, d = e % DP;
    sE[vv * DPE + d] = (vv < rows && d < p.D) ? E[(int64_t)(vg0 + vv) * p.lde + d] : (T)0.f;
  }
  if ((int)threadIdx.x < BV) {
    const int vv = threadIdx.x;
    sBias[vv] = vv < rows ? (p.bias ? p.bias[vg0 + vv] : 0.f) : kNegInf;
  }

  f32x16_t deacc[DB][FV];
  float dbacc[FV];
#pragma unroll
  for (int fv = 0; fv < FV; ++fv) {
    dbacc[fv] = 0.f;
#pragma unroll
    for (int db = 0; db < DB; ++db) deacc[db][fv] = zero16();
  }

  KTile<T, BM, kBK> th;
  th.ld = p.ldh;
  th.k_valid = p.K;
  KTile<T, BV, kBK> tw;
  tw.base = static_cast<const T*>(p.W) + (int64_t)vg0 * p.ldw;
  tw.ld = p.ldw;
  tw.rows_valid = rows;
  tw.k_valid = p.K;
  const int nk = (p.K + kBK - 1) / kBK;
  T* stage = static_cast<T*>(p.stage);

  for (int tb = tb_begin; tb < tb_end; ++tb) {
    const int n0 = tb * BM;
    th.base = static_cast<const T*>(p.h) + (int64_t)n0 * p.ldh;
    th.rows_valid = p.N - n0;
    ScoresSide<T, BM, DP, DPE> side;
    side.sG = sG;
    side.sLse = sLse;
    side.sDelta = sDelta;
    side.gO = p.gO;
    side.lse = p.lse;
    side.delta = p.delta;
    side.n0 = n0;
    side.N = p.N;
    side.D = p.D;

    f32x16_t sacc[FT][FV];
#pragma unroll
    for (int ft = 0; ft < FT; ++ft)
#pragma unroll
      for (int fv = 0; fv < FV; ++fv) sacc[ft][fv] = zero16();
    reduce_loop<T, kBK, FT, FV>(sacc, th, tw, sH[0], sH[1], sW[0], sW[1], p.K, 0, w * WVR, side);
    side.finish(nk);

#pragma unroll
    for (int fv = 0; fv < FV; ++fv) {
      const int vl = w * WVR + fv * 32 + (lane & 31);  // tile-local row of this lane
      const float bvv = sBias[vl];
#pragma unroll
      for (int ft = 0; ft < FT; ++ft) {
        // dP block = gO[tokens] E[rows]^T over D
        f32x16_t dp = zero16();
#pragma unroll
        for (int kd = 0; kd < DK; ++kd) {
          const V8 a = *reinterpret_cast<const V8*>(sG + (ft * 32 + (lane & 31)) * DPE + kd * 16 + (lane >> 5) * 8);
          const V8 b = *reinterpret_cast<const V8*>(sE + vl * DPE + kd * 16 + (lane >> 5) * 8);
          mfma_k16(dp, a, b);
        }
        float dbs = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int tl = ft * 32 + c_row(r, lane);
          const float x = sacc[ft][fv][r] * p.scale + bvv;
          const float pv = fast_exp(x - sLse[tl]);
          const float ds = pv * (dp[r] - sDelta[tl]);
          dbs += ds;
          sacc[ft][fv][r] = pv;
          dp[r] = ds * p.scale;  // dL/d(h W^T) (swvr/chunked.py:143-144)
        }
        dbacc[fv] += dbs;
        if (p.need_stage) {
          T* dst = stage + (int64_t)(vl0 + vl) * p.ld_stage + n0 + ft * 32 + (lane >> 5) * 4;
#pragma unroll
          for (int g4 = 0; g4 < 4; ++g4) {
            if constexpr (sizeof(T) == 2) {
              T q[4];
#pragma unroll
              for (int i = 0; i < 4; ++i) q[i] = from_float<T>(dp[4 * g4 + i]);
              uint2 u;
              __builtin_memcpy(&u, q, 8);
              *reinterpret_cast<uint2*>(dst + g4 * 8) = u;
            } else {
              *reinterpret_cast<float4*>(dst + g4 * 8) =
                  make_float4(dp[4 * g4], dp[4 * g4 + 1], dp[4 * g4 + 2], dp[4 * g4 + 3]);
            }
          }
        }
        if (p.need_dE) {
          // dE^T[d][v] += gO^T[d][tok] P[tok][v]; registers 8c..8c+7 hold
          // tokens 16c + 8(t/4) + 4(lane/32) + t%4, gathered likewise from sG
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            V8 bv;
#pragma unroll
            for (int tt = 0; tt < 8; ++tt) bv[tt] = from_float<T>(sacc[ft][fv][8 * c + tt]);
#pragma unroll
            for (int db = 0; db < DB; ++db) {
              V8 av;
#pragma unroll
              for (int tt = 0; tt < 8; ++tt) {
                const int tl = ft * 32 + 16 * c + 8 * (tt >> 2) + (lane >> 5) * 4 + (tt & 3);
                av[tt] = sG[tl * DPE + db * 32 + (lane & 31)];
              }
              mfma_k16(deacc[db][fv], av, bv);
            }
          }
        }
      }
    }
  }

#pragma unroll
  for (int fv = 0; fv < FV; ++fv) {
    const int vc = vl0 + w * WVR + fv * 32 + (lane & 31);  // chunk-local row
    if (p.need_db) {
      const float s = wave_sum32(dbacc[fv]);
      if (lane < 32) p.part_db[(int64_t)g * p.C + vc] = s;
    }
    if (p.need_dE) {
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int d = db * 32 + c_row(r, lane);
          p.part_dE[((int64_t)g * DP + d) * p.C + vc] = deacc[db][fv][r];
        }
    }
  }
}

// ---------------------------------------------------------------- GEMMs
struct GemmParams {
  const void* stage;
  int64_t ld_stage;
  int64_t N_pad;
  const void* h;
  int64_t ldh;
  const void* W;
  int64_t ldw;
  int N, K;
  int v0, cv;
  int n_n;         // tiles along K
  int n_dw, n_dh;  // tile counts (0 when that gradient is not needed)
  void* gW;
  int gW_dtype;
  float* dh_acc;
  void* gh;
  int gh_dtype;
  int dh_first, dh_last;
};

// One launch covers both gradient products of a chunk:
//   blocks [0, n_dw):          dW[v0+v][k]  = sum_tok stage[v][tok] h[tok][k]
//   blocks [n_dw, n_dw+n_dh):  dh[tok][k] += sum_v  stage[v][tok] W[v0+v][k]
// The dW tiles (the longer reduction) are dealt first.
template <class T, int GM, int GN>
__global__ __launch_bounds__(kThreads) void bwd_gemm_kernel(GemmParams p) {
  constexpr int FM = GM / 64, FN = GN / 64;
  constexpr int LDR = LdsRow<T, kBK>::value;
  __shared__ __attribute__((aligned(16))) T sA[2][GM * LDR];
  __shared__ __attribute__((aligned(16))) T sB[2][GN * LDR];

  const int lane = lane_id(), w = wave_id();
  const int wm = w >> 1, wn = w & 1;
  const T* stage = static_cast<const T*>(p.stage);
  f32x16_t acc[FM][FN];
#pragma unroll
  for (int fm = 0; fm < FM; ++fm)
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) acc[fm][fn] = zero16();
  NoSide none;
  const int b = blockIdx.x;
  if (b < p.n_dw) {
    const int t = xcd_swizzle(b, p.n_dw);
    const int mt = t / p.n_n, nt = t % p.n_n;
    KTile<T, GM, kBK> ta;
    ta.base = stage + (int64_t)mt * GM * p.ld_stage;
    ta.ld = p.ld_stage;
    ta.rows_valid = p.cv - mt * GM;
    ta.k_valid = (int)p.N_pad;
    RTile<T, GN, kBK> tb;
    tb.base = static_cast<const T*>(p.h) + nt * GN;
    tb.ld = p.ldh;
    tb.rows_valid = p.K - nt * GN;
    tb.k_valid = p.N;
    reduce_loop<T, kBK, FM, FN>(acc, ta, tb, sA[0], sA[1], sB[0], sB[1], p.N, wm * (GM / 2), wn * (GN / 2), none);
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) {
        const int col = nt * GN + wn * (GN / 2) + fn * 32 + (lane & 31);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = mt * GM + wm * (GM / 2) + fm * 32 + c_row(r, lane);
          if (row < p.cv && col < p.K) store_as(p.gW, (int64_t)(p.v0 + row) * p.K + col, p.gW_dtype, acc[fm][fn][r]);
        }
      }
  } else {
    const int t = xcd_swizzle(b - p.n_dw, p.n_dh);
    const int mt = t / p.n_n, nt = t % p.n_n;
    RTile<T, GM, kBK> ta;
    ta.base = stage + (int64_t)mt * GM;
    ta.ld = p.ld_stage;
    ta.rows_valid = (int)(p.N_pad - (int64_t)mt * GM);
    ta.k_valid = p.cv;
    RTile<T, GN, kBK> tb;
    tb.base = static_cast<const T*>(p.W) + (int64_t)p.v0 * p.ldw + nt * GN;
    tb.ld = p.ldw;
    tb.rows_valid = p.K - nt * GN;
    tb.k_valid = p.cv;
    reduce_loop<T, kBK, FM, FN>(acc, ta, tb, sA[0], sA[1], sB[0], sB[1], p.cv, wm * (GM / 2), wn * (GN / 2), none);
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) {
        const int col = nt * GN + wn * (GN / 2) + fn * 32 + (lane & 31);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = mt * GM + wm * (GM / 2) + fm * 32 + c_row(r, lane);
          if (row < p.N && col < p.K) {
            const int64_t idx = (int64_t)row * p.K + col;
            float v = acc[fm][fn][r];
            if (!p.dh_first) v += p.dh_acc[idx];
            if (p.dh_last)
              store_as(p.gh, idx, p.gh_dtype, v);
            else
              p.dh_acc[idx] = v;
          }
        }
      }
  }
}

// ---------------------------------------------------------------- dE / db
__global__ __launch_bounds__(256) void bwd_reduce_kernel(const float* __restrict__ part_dE,
                                                         const float* __restrict__ part_db, int G, int C, int DP,
                                                         int v0, int cv, int D, void* gE, int gE_dtype,
                                                         float* gb) {
  const int v = blockIdx.x * blockDim.x + threadIdx.x;
  if (v >= cv) return;
  if (gE) {
    for (int d = 0; d < D; ++d) {
      float s = 0.f;
      for (int g = 0; g < G; ++g) s += part_dE[((int64_t)g * DP + d) * C + v];
      store_as(gE, (int64_t)(v0 + v) * D + d, gE_dtype, s);
    }
  }
  if (gb) {
    float s = 0.f;
    for (int g = 0; g < G; ++g) s += part_db[(int64_t)g * C + v];
    gb[v0 + v] = s;
  }
}

// Zero fill with a kernel (not hipMemsetAsync), so a caller may capture it in
// a graph.  Buffers here hold whole 2- or 4-byte elements.
__global__ __launch_bounds__(256) void fill_zero_kernel(uint16_t* p, int64_t n_halves) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_halves;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0;
}

hipError_t fill_zero(void* p, size_t bytes, hipStream_t stream) {
  if (!p || bytes == 0) return hipSuccess;
  const int64_t halves = (int64_t)(bytes / 2);
  const int blocks = (int)((halves + 255) / 256 < 4096 ? (halves + 255) / 256 : 4096);
  timing_begin(kKindFill, stream);
  fill_zero_kernel<<<blocks, 256, 0, stream>>>(static_cast<uint16_t*>(p), halves);
  timing_end(kKindFill, stream);
  return hipGetLastError();
}

template <class T, int BM, int BV, int DP>
hipError_t launch_scores(const ScoresParams& sp, hipStream_t stream) {
  timing_begin(kKindBwdScores, stream);
  bwd_scores_kernel<T, BM, BV, DP><<<sp.n_vtc * sp.G, kThreads, 0, stream>>>(sp);
  timing_end(kKindBwdScores, stream);
  return hipGetLastError();
}

// Tile shape of the scores kernel per (dtype, padded D): dE^T (DP x BV/4 per
// wave) and the score block (BM x BV/4 per wave) share the register file; E,
// the gO tile and two K-slices of h and W share LDS.
template <class T, int DP>
struct ScoresTile {
  static constexpr bool wide = sizeof(T) == 2;
  static constexpr int BM = wide ? (DP <= 128 ? 128 : 64) : 64;
  static constexpr int BV = wide ? (DP <= 64 ? 256 : 128) : 128;
};

template <class T>
struct GemmTile {
  static constexpr int GM = sizeof(T) == 2 ? 256 : 128;
  static constexpr int GN = GM;
};

template <class T, int DP>
hipError_t dispatch_scores_tile(const BwdPlan& plan, const ScoresParams& sp, hipStream_t stream) {
  typedef ScoresTile<T, DP> C;
  if (plan.BM != C::BM || plan.BV != C::BV) return hipErrorInvalidValue;
  return launch_scores<T, C::BM, C::BV, DP>(sp, stream);
}

template <class T>
hipError_t dispatch_scores(const BwdPlan& plan, const ScoresParams& sp, hipStream_t stream) {
  switch (plan.DP) {
    case 32: return dispatch_scores_tile<T, 32>(plan, sp, stream);
    case 64: return dispatch_scores_tile<T, 64>(plan, sp, stream);
    case 128: return dispatch_scores_tile<T, 128>(plan, sp, stream);
    case 256:
      if constexpr (sizeof(T) == 2) return dispatch_scores_tile<T, 256>(plan, sp, stream);
      return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
}

template <class T>
hipError_t dispatch_gemm(const BwdPlan& plan, const GemmParams& gp, hipStream_t stream) {
  const int blocks = gp.n_dw + gp.n_dh;
  if (blocks == 0) return hipSuccess;
  if (plan.GM != GemmTile<T>::GM || plan.GN != GemmTile<T>::GN) return hipErrorInvalidValue;
  timing_begin(kKindBwdGemm, stream);
  bwd_gemm_kernel<T, GemmTile<T>::GM, GemmTile<T>::GN><<<blocks, kThreads, 0, stream>>>(gp);
  timing_end(kKindBwdGemm, stream);
  return hipGetLastError();
}

template <class T>
hipError_t bwd_run(const BwdPlan& plan, const BwdParams& p, hipStream_t stream) {
  hipError_t e;
  char* ws = p.ws;
  float* delta = reinterpret_cast<float*>(ws + plan.off_delta);
  T* stage = reinterpret_cast<T*>(ws + plan.off_stage);
  float* part_dE = reinterpret_cast<float*>(ws + plan.off_pe);
  float* part_db = reinterpret_cast<float*>(ws + plan.off_pb);
  float* dh_acc = plan.dh_acc ? reinterpret_cast<float*>(ws + plan.off_dh) : nullptr;

  timing_begin(kKindBwdDelta, stream);
  bwd_delta_kernel<<<(p.N + 255) / 256, 256, 0, stream>>>(p.O, p.gO, p.glse, p.N, p.D, delta);
  timing_end(kKindBwdDelta, stream);
  if ((e = hipGetLastError()) != hipSuccess) return e;

  const bool need_stage = p.gh || p.gW;
  for (int c = 0; c < plan.n_chunks; ++c) {
    const int v0 = (int)(c * plan.C);
    const int cv = (int)((p.V - v0) < plan.C ? (p.V - v0) : plan.C);
    ScoresParams sp;
    sp.h = p.h;
    sp.ldh = p.ldh;
    sp.W = p.W;
    sp.ldw = p.ldw;
    sp.E = p.E;
    sp.lde = p.lde;
    sp.bias = p.bias;
    sp.scale = p.scale;
    sp.N = p.N;
    sp.K = p.K;
    sp.D = p.D;
    sp.lse = p.lse;
    sp.delta = delta;
    sp.gO = p.gO;
    sp.v0 = v0;
    sp.cv = cv;
    sp.C = (int)plan.C;
    sp.n_tb = plan.n_tb;
    sp.G = plan.G;
    sp.n_vtc = (cv + plan.BV - 1) / plan.BV;
    sp.stage = stage;
    sp.ld_stage = plan.N_pad;
    sp.part_dE = part_dE;
    sp.part_db = part_db;
    sp.need_stage = need_stage;
    sp.need_dE = p.gE != nullptr;
    sp.need_db = p.gb != nullptr;
    if ((e = dispatch_scores<T>(plan, sp, stream)) != hipSuccess) return e;

    if (need_stage) {
      GemmParams gp;
      gp.stage = stage;
      gp.ld_stage = plan.N_pad;
      gp.N_pad = plan.N_pad;
      gp.h = p.h;
      gp.ldh = p.ldh;
      gp.W = p.W;
      gp.ldw = p.ldw;
      gp.N = p.N;
      gp.K = p.K;
      gp.v0 = v0;
      gp.cv = cv;
      gp.n_n = (p.K + plan.GN - 1) / plan.GN;
      gp.n_dw = p.gW ? ((cv + plan.GM - 1) / plan.GM) * gp.n_n : 0;
      gp.n_dh = p.gh ? ((p.N + plan.GM - 1) / plan.GM) * gp.n_n : 0;
      gp.gW = p.gW;
      gp.gW_dtype = p.gW_dtype;
      gp.dh_acc = dh_acc;
      gp.gh = p.gh;
      gp.gh_dtype = p.gh_dtype;
      gp.dh_first = c == 0;
      gp.dh_last = c == plan.n_chunks - 1;
      if ((e = dispatch_gemm<T>(plan, gp, stream)) != hipSuccess) return e;
    }
    if (p.gE || p.gb) {
      timing_begin(kKindBwdReduce, stream);
      bwd_reduce_kernel<<<(cv + 255) / 256, 256, 0, stream>>>(part_dE, part_db, plan.G, (int)plan.C, plan.DP, v0, cv,
                                                              p.D, p.gE, p.gE_dtype, p.gb);
      timing_end(kKindBwdReduce, stream);
      if ((e = hipGetLastError()) != hipSuccess) return e;
    }
  }
  return hipSuccess;
}

template <class T>
void scores_tile_of(int DP, int* BM, int* BV) {
  switch (DP) {
    case 32: *BM = ScoresTile<T, 32>::BM; *BV = ScoresTile<T, 32>::BV; break;
    case 64: *BM = ScoresTile<T, 64>::BM; *BV = ScoresTile<T, 64>::BV; break;
    case 128: *BM = ScoresTile<T, 128>::BM; *BV = ScoresTile<T, 128>::BV; break;
    default: *BM = ScoresTile<T, 256>::BM; *BV = ScoresTile<T, 256>::BV; break;
  }
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

size_t dtype_bytes(int dtype) { return dtype == kF32 ? 4 : 2; }

}  // namespace

bool bwd_plan(int dtype, int64_t N, int64_t K, int64_t V, int64_t D, int64_t chunk, bool need_gh, BwdPlan* plan) {
  const int DP = D <= 32 ? 32 : D <= 64 ? 64 : D <= 128 ? 128 : D <= 256 ? 256 : 0;
  if (DP == 0) return false;
  int BM, BV, GM, GN;
  if (dtype == kF32) {
    if (DP > 128) return false;
    scores_tile_of<float>(DP, &BM, &BV);
    GM = GemmTile<float>::GM;
    GN = GemmTile<float>::GN;
  } else if (dtype == kBF16 || dtype == kF16) {
    scores_tile_of<bf16_t>(DP, &BM, &BV);
    GM = GemmTile<bf16_t>::GM;
    GN = GemmTile<bf16_t>::GN;
  } else {
    return false;
  }
  plan->DP = DP;
  plan->BM = BM;
  plan->BV = BV;
  plan->GM = GM;
  plan->GN = GN;
  plan->n_tb = (int)((N + BM - 1) / BM);
  plan->N_pad = ((N + 255) / 256) * 256;
  if (plan->N_pad == 0) plan->N_pad = 256;
  int64_t c = chunk < V ? chunk : V;
  if (c < 1) c = 1;
  c = ((c + BV - 1) / BV) * BV;
  plan->C = c;
  plan->n_chunks = (int)((V + c - 1) / c);
  const int n_vtc = (int)(c / BV);
  int G = (512 + n_vtc - 1) / n_vtc;
  if (G > plan->n_tb) G = plan->n_tb;
  if (G < 1) G = 1;
  plan->G = G;
  plan->dh_acc = need_gh && plan->n_chunks > 1;
  size_t off = 0;
  plan->off_delta = off;
  off += align256((size_t)N * 4);
  plan->off_stage = off;
  off += align256((size_t)c * (size_t)plan->N_pad * dtype_bytes(dtype));
  plan->off_pe = off;
  off += align256((size_t)G * DP * c * 4);
  plan->off_pb = off;
  off += align256((size_t)G * c * 4);
  plan->off_dh = off;
  if (plan->dh_acc) off += align256((size_t)N * K * 4);
  plan->ws_bytes = off;
  return true;
}

hipError_t bwd_launch(int dtype, const BwdPlan& plan, const BwdParams& p, hipStream_t stream) {
  if (p.N == 0) {
    // no tokens: every gradient of the vocabulary side is zero
    hipError_t e;
    if ((e = fill_zero(p.gW, (size_t)p.V * p.K * dtype_bytes(p.gW_dtype), stream)) != hipSuccess) return e;
    if ((e = fill_zero(p.gE, (size_t)p.V * p.D * dtype_bytes(p.gE_dtype), stream)) != hipSuccess) return e;
    if ((e = fill_zero(p.gb, (size_t)p.V * 4, stream)) != hipSuccess) return e;
    return hipSuccess;
  }
  switch (dtype) {
    case kBF16: return bwd_run<bf16_t>(plan, p, stream);
    case kF16: return bwd_run<f16_t>(plan, p, stream);
    case kF32: return bwd_run<float>(plan, p, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace swvr
