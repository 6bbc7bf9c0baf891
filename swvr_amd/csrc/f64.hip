// The readout in fp64 (the reference's precision for fp64 inputs:
// swvr/chunked.py:26-27 accumulates and returns fp64 when the compute dtype is
// fp64, on its torch path, swvr/chunked.py:62-63).
//
// gfx950's matrix cores serve fp64 only at the rate of its vector units, and
// fp64 readouts are checking and small-model work, so this path favours
// exactness and simplicity: the reference's vocabulary-chunked algorithm
// (swvr/chunked.py:82-151) over a strided fp64 GEMM tiled through LDS, plus
// row-wise softmax kernels.  Every reduction has a fixed order, so results are
// reproducible bit for bit.
//
// forward, per chunk [v0, v0 + C):   S = s h W_c^T + b_c                      (gemm)
//                                    m, l, acc <- online softmax of S, P = e^(S - m)
//                                    acc += P E_c                             (gemm)
//            then O = acc / l, lse = m + log l
// backward: delta = rowsum(O gO) - glse; per chunk:
//            S (gemm), P = e^(S - lse), dP = gO E_c^T (gemm), dS = P (dP - delta),
//            gb_c = colsum dS, gE_c = P^T gO, gh += s dS W_c, gW_c = s dS^T h  (gemms)
#include <math.h>

#include "common.hpp"
#include "launch.hpp"

namespace swvr {

namespace {

constexpr int kTile = 64;   // output tile per workgroup (kTile x kTile)
constexpr int kSlice = 16;  // reduction slice staged in LDS

// C[m][n] = alpha * sum_k A(m, k) B(k, n) (+ beta * C[m][n] when beta != 0) (+ colv[n]),
// with A(m, k) = A[m sam + k sak], B(k, n) = B[k sbk + n sbn], C rows ldc apart.
// 256 threads, each 4 x 4 outputs (rows tm + 16 i, columns tn + 16 j).  Operand
// loads walk the unit-stride dimension across consecutive threads when there is one.
__global__ __launch_bounds__(256) void gemm_f64_kernel(int M, int N, int K, const double* __restrict__ A,
                                                       int64_t sam, int64_t sak, const double* __restrict__ B,
                                                       int64_t sbk, int64_t sbn, double alpha, double beta,
                                                       const double* __restrict__ colv, double* __restrict__ C,
                                                       int64_t ldc) {
  __shared__ double As[kSlice][kTile + 1];  // [k][m]
  __shared__ double Bs[kSlice][kTile + 1];  // [k][n]
  const int tid = threadIdx.x;
  const int tm = tid / 16, tn = tid % 16;
  const int m0 = blockIdx.x * kTile, n0 = blockIdx.y * kTile;
  const bool a_kfast = sak == 1, b_kfast = sbk == 1;
  double acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.0;
  for (int k0 = 0; k0 < K; k0 += kSlice) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = i * 256 + tid;  // element of the 64 x 16 operand tile
      const int ak = a_kfast ? e % kSlice : e / kTile, am = a_kfast ? e / kSlice : e % kTile;
      const int m = m0 + am, k = k0 + ak;
      As[ak][am] = (m < M && k < K) ? A[(int64_t)m * sam + (int64_t)k * sak] : 0.0;
      const int bk = b_kfast ? e % kSlice : e / kTile, bn = b_kfast ? e / kSlice : e % kTile;
      const int n = n0 + bn, k2 = k0 + bk;
      Bs[bk][bn] = (n < N && k2 < K) ? B[(int64_t)k2 * sbk + (int64_t)n * sbn] : 0.0;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kSlice; ++kk) {
      double a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = As[kk][tm + 16 * i];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = Bs[kk][tn + 16 * j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fma(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = m0 + tm + 16 * i;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + tn + 16 * j;
      if (n >= N) continue;
      double* c = C + (int64_t)m * ldc + n;
      double v = alpha * acc[i][j];
      if (beta != 0.0) v += beta * *c;
      if (colv) v += colv[n];
      *c = v;
    }
  }
}

hipError_t gemm(int M, int N, int K, const double* A, int64_t sam, int64_t sak, const double* B, int64_t sbk,
                int64_t sbn, double alpha, double beta, const double* colv, double* C, int64_t ldc,
                hipStream_t stream) {
  if (M <= 0 || N <= 0) return hipSuccess;
  const dim3 grid((M + kTile - 1) / kTile, (N + kTile - 1) / kTile);  // N / 64 <= 65535: N < 2^22
  gemm_f64_kernel<<<grid, 256, 0, stream>>>(M, N, K, A, sam, sak, B, sbk, sbn, alpha, beta, colv, C, ldc);
  return hipGetLastError();
}

__global__ __launch_bounds__(256) void fill_f64_kernel(double* p, int64_t n, double v) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = v;
}

hipError_t fill(double* p, int64_t n, double v, hipStream_t stream) {
  if (!p || n <= 0) return hipSuccess;
  const int64_t blocks = (n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096;
  fill_f64_kernel<<<(unsigned)blocks, 256, 0, stream>>>(p, n, v);
  return hipGetLastError();
}

// Block-wide reduction in a fixed order (256 threads): op over v, result in every thread.
template <class Op>
__device__ double block_reduce(double v, double* sh, Op op) {
  sh[threadIdx.x] = v;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) sh[threadIdx.x] = op(sh[threadIdx.x], sh[threadIdx.x + s]);
    __syncthreads();
  }
  const double r = sh[0];
  __syncthreads();
  return r;
}

// One row per workgroup: the online-softmax update of swvr/chunked.py:96-104 over the
// chunk's scores S[n][0:cv] (replaced by P = e^(S - shift)), m[n], l[n] and acc[n][0:D].
__global__ __launch_bounds__(256) void online_f64_kernel(double* __restrict__ S, int cv, double* __restrict__ m,
                                                         double* __restrict__ l, double* __restrict__ acc, int D) {
  __shared__ double sh[256];
  const int64_t n = blockIdx.x;
  double* row = S + n * cv;
  double mx = -HUGE_VAL;
  for (int v = threadIdx.x; v < cv; v += 256) mx = fmax(mx, row[v]);
  mx = block_reduce(mx, sh, [](double a, double b) { return fmax(a, b); });
  const double m_old = m[n];
  const double m_new = fmax(m_old, mx);
  const double shift = m_new == -HUGE_VAL ? 0.0 : m_new;  // a row of -inf so far: shift by 0
  const double alpha = exp(m_old - shift);
  double sum = 0.0;
  for (int v = threadIdx.x; v < cv; v += 256) {
    const double p = exp(row[v] - shift);
    row[v] = p;
    sum += p;
  }
  sum = block_reduce(sum, sh, [](double a, double b) { return a + b; });
  for (int d = threadIdx.x; d < D; d += 256) acc[n * D + d] *= alpha;
  if (threadIdx.x == 0) {
    m[n] = m_new;
    l[n] = l[n] * alpha + sum;
  }
}

// O = acc / l and lse = m + log l (swvr/chunked.py:105).
__global__ __launch_bounds__(256) void finish_f64_kernel(const double* __restrict__ acc, const double* __restrict__ m,
                                                         const double* __restrict__ l, int N, int D,
                                                         double* __restrict__ O, double* __restrict__ lse) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int Dw = D > 0 ? D : 1;
  if (e >= (int64_t)N * Dw) return;
  const int64_t n = e / Dw;
  const int d = (int)(e % Dw);
  if (d < D) O[e] = acc[e] / l[n];
  if (d == 0) lse[n] = m[n] + log(l[n]);
}

// delta = rowsum(O gO) - glse (swvr/chunked.py:113-114), one thread per row.
__global__ __launch_bounds__(256) void delta_f64_kernel(const double* __restrict__ O, const double* __restrict__ gO,
                                                        const double* __restrict__ glse, int N, int D,
                                                        double* __restrict__ delta) {
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  double s = 0.0;
  for (int d = 0; d < D; ++d) s += O[n * D + d] * gO[n * D + d];
  delta[n] = s - glse[n];
}

// P = e^(S - lse) in place, dS = P (dP - delta) in place (swvr/chunked.py:133-139).
__global__ __launch_bounds__(256) void softmax_bwd_f64_kernel(double* __restrict__ S, double* __restrict__ dP, int N,
                                                              int cv, const double* __restrict__ lse,
                                                              const double* __restrict__ delta) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= (int64_t)N * cv) return;
  const int64_t n = e / cv;
  const double p = exp(S[e] - lse[n]);
  S[e] = p;
  dP[e] = p * (dP[e] - delta[n]);
}

// gb[v] = sum_n dS[n][v], one thread per column, rows in order.
__global__ __launch_bounds__(256) void colsum_f64_kernel(const double* __restrict__ dS, int N, int cv,
                                                         double* __restrict__ gb) {
  const int v = blockIdx.x * blockDim.x + threadIdx.x;
  if (v >= cv) return;
  double s = 0.0;
  for (int64_t n = 0; n < N; ++n) s += dS[n * cv + v];
  gb[v] = s;
}

}  // namespace

void f64_plan(int64_t N, int64_t V, int64_t D, int64_t chunk, int64_t* C, size_t* fwd_bytes, size_t* bwd_bytes) {
  int64_t c = chunk < V ? chunk : V;
  if (c > ((int64_t)1 << 22)) c = (int64_t)1 << 22;  // the chunk's columns are one grid dimension of a GEMM
  if (c < 1) c = 1;
  *C = c;
  const size_t a = 256;
  auto al = [a](size_t x) { return (x + a - 1) / a * a; };
  const size_t chunk_bytes = al((size_t)N * (size_t)c * sizeof(double));
  if (fwd_bytes) *fwd_bytes = chunk_bytes + 2 * al((size_t)N * sizeof(double)) + al((size_t)N * D * sizeof(double));
  if (bwd_bytes) *bwd_bytes = 2 * chunk_bytes + al((size_t)N * sizeof(double));
}

hipError_t f64_fwd(const F64Params& p, hipStream_t stream) {
  int64_t C;
  size_t fb;
  f64_plan(p.N, p.V, p.D, p.chunk, &C, &fb, nullptr);
  const size_t chunk_bytes = ((size_t)p.N * (size_t)C * sizeof(double) + 255) / 256 * 256;
  const size_t row_bytes = ((size_t)p.N * sizeof(double) + 255) / 256 * 256;
  double* S = reinterpret_cast<double*>(p.ws);
  double* m = reinterpret_cast<double*>(p.ws + chunk_bytes);
  double* l = reinterpret_cast<double*>(p.ws + chunk_bytes + row_bytes);
  double* acc = reinterpret_cast<double*>(p.ws + chunk_bytes + 2 * row_bytes);
  hipError_t e;
  timing_begin(kKindF64, stream);
  if ((e = fill(m, p.N, -HUGE_VAL, stream)) != hipSuccess) return e;
  if ((e = fill(l, p.N, 0.0, stream)) != hipSuccess) return e;
  if ((e = fill(acc, (int64_t)p.N * p.D, 0.0, stream)) != hipSuccess) return e;
  for (int64_t v0 = 0; v0 < p.V; v0 += C) {
    const int cv = (int)(p.V - v0 < C ? p.V - v0 : C);
    // S = s h W_c^T + b_c
    if ((e = gemm(p.N, cv, p.K, p.h, p.ldh, 1, p.W + v0 * p.ldw, 1, p.ldw, p.scale, 0.0, p.bias ? p.bias + v0 : nullptr,
                  S, cv, stream)) != hipSuccess)
      return e;
    online_f64_kernel<<<p.N, 256, 0, stream>>>(S, cv, m, l, acc, p.D);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    // acc += P E_c
    if ((e = gemm(p.N, p.D, cv, S, cv, 1, p.E + v0 * p.lde, p.lde, 1, 1.0, 1.0, nullptr, acc, p.D, stream)) !=
        hipSuccess)
      return e;
  }
  const int64_t nt = (int64_t)p.N * (p.D > 0 ? p.D : 1);
  finish_f64_kernel<<<(unsigned)((nt + 255) / 256), 256, 0, stream>>>(acc, m, l, p.N, p.D, p.O, p.lse);
  timing_end(kKindF64, stream);
  return hipGetLastError();
}

hipError_t f64_bwd(const F64Params& p, hipStream_t stream) {
  if (p.N == 0) {
    // no tokens: every gradient of the vocabulary side is zero (the workspace is not used)
    hipError_t e;
    if ((e = fill(p.gW, (int64_t)p.V * p.K, 0.0, stream)) != hipSuccess) return e;
    if ((e = fill(p.gE, (int64_t)p.V * p.D, 0.0, stream)) != hipSuccess) return e;
    return fill(p.gb, p.V, 0.0, stream);
  }
  int64_t C;
  size_t bb;
  f64_plan(p.N, p.V, p.D, p.chunk, &C, nullptr, &bb);
  const size_t chunk_bytes = ((size_t)p.N * (size_t)C * sizeof(double) + 255) / 256 * 256;
  double* S = reinterpret_cast<double*>(p.ws);
  double* dP = reinterpret_cast<double*>(p.ws + chunk_bytes);
  double* delta = reinterpret_cast<double*>(p.ws + 2 * chunk_bytes);
  hipError_t e;
  timing_begin(kKindF64, stream);
  delta_f64_kernel<<<(unsigned)((p.N + 255) / 256), 256, 0, stream>>>(p.O, p.gO, p.glse, p.N, p.D, delta);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  if ((e = fill(p.gh, (int64_t)p.N * p.K, 0.0, stream)) != hipSuccess) return e;
  for (int64_t v0 = 0; v0 < p.V; v0 += C) {
    const int cv = (int)(p.V - v0 < C ? p.V - v0 : C);
    // S = s h W_c^T + b_c, dP = gO E_c^T
    if ((e = gemm(p.N, cv, p.K, p.h, p.ldh, 1, p.W + v0 * p.ldw, 1, p.ldw, p.scale, 0.0, p.bias ? p.bias + v0 : nullptr,
                  S, cv, stream)) != hipSuccess)
      return e;
    if ((e = gemm(p.N, cv, p.D, p.gO, p.D, 1, p.E + v0 * p.lde, 1, p.lde, 1.0, 0.0, nullptr, dP, cv, stream)) !=
        hipSuccess)
      return e;
    const int64_t ne = (int64_t)p.N * cv;
    softmax_bwd_f64_kernel<<<(unsigned)((ne + 255) / 256), 256, 0, stream>>>(S, dP, p.N, cv, p.lse, delta);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if (p.gb) {
      colsum_f64_kernel<<<(cv + 255) / 256, 256, 0, stream>>>(dP, p.N, cv, p.gb + v0);
      if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    // gE_c = P^T gO
    if (p.gE && (e = gemm(cv, p.D, p.N, S, 1, cv, p.gO, p.D, 1, 1.0, 0.0, nullptr, p.gE + v0 * p.D, p.D, stream)) !=
                    hipSuccess)
      return e;
    // gh += s dS W_c
    if (p.gh && (e = gemm(p.N, p.K, cv, dP, cv, 1, p.W + v0 * p.ldw, p.ldw, 1, p.scale, 1.0, nullptr, p.gh, p.K,
                          stream)) != hipSuccess)
      return e;
    // gW_c = s dS^T h
    if (p.gW && (e = gemm(cv, p.K, p.N, dP, 1, cv, p.h, p.ldh, 1, p.scale, 0.0, nullptr, p.gW + v0 * p.K, p.K,
                          stream)) != hipSuccess)
      return e;
  }
  timing_end(kKindF64, stream);
  return hipSuccess;
}

}  // namespace swvr
