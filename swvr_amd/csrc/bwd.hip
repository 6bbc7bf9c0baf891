// Backward of the readout (docs/DESIGN.md:26-37, swvr/chunked.py:108-151).
//
//   delta = rowsum(O * gO) - gLSE                                 bwd_delta_kernel
//   per vocabulary chunk [v0, v0 + C):
//     P  = exp(s * h W_c^T + b_c - LSE)        (scores recomputed)
//     dS = P * (gO E_c^T - delta)                                 the scores kernels
//       -> stage dS in the compute dtype, in 32 x 32 blocks (what the gradient GEMMs consume,
//          swvr/chunked.py:143-145 / triton_kernels.py:108-109; the
//          reference stages s*dS, here the GEMMs apply s to their outputs)
//       -> dE_c = P^T gO and db_c = colsum(dS), accumulated per token group
//          in registers and written as partials (no atomics)
//     dW_c = s stage^T h   and   dh += s stage W_c                bwd_gemm_kernel
//     dE_c, db_c = fixed-order sum of the partials                workgroups after the GEMM
//                                                                 tiles of the same launch
//                                                                 (bwd_reduce_kernel when
//                                                                 neither gW nor gh is needed)
//     W_{c+1} packed for the next scores launch                   workgroups after those
//   Wide embeddings (bwd_scores_wide_kernel) keep no dE accumulator: the scores
//   kernel also stages P, dE_c^T = gO^T P is a product of the GEMM launch, and
//   bwd_reduce_kernel sums the db partials and writes gE from dE_c^T.
// Every reduction has a fixed order, so gradients are bitwise reproducible.
#include <type_traits>

#include "common.hpp"
#include "launch.hpp"

namespace swvr {

namespace {

__device__ __forceinline__ void store_as(void* base, int64_t idx, int dtype, float v) {
  if (dtype == kBF16)
    static_cast<bf16_t*>(base)[idx] = (bf16_t)v;
  else if (dtype == kF16)
    static_cast<f16_t*>(base)[idx] = (f16_t)v;
  else
    static_cast<float*>(base)[idx] = v;
}

// ---------------------------------------------------------------- token-side packing
// The backward runs over the active tokens only: a token whose cotangents are
// all zero (gO row = 0, gLSE = 0, so delta = 0) has dS = P (dP - delta) = 0
// in every vocabulary row, so it adds nothing to gW, gE or gb and its gh row
// is zero.  (A token with a non-finite O has a NaN delta and stays active, as
// the reference propagates it.)  Zero-weight tokens of a weighted loss are
// such tokens.  The active tokens are compacted in ascending order into
// positions 0 .. n_act - 1; positions n_act .. N_pad - 1 are padding.

// delta = rowsum(O * gO) - gLSE (swvr/chunked.py:113-114) and the active flag,
// one thread per token.  gO enters the sum rounded to the compute dtype T, as it
// enters dP = gO E^T: the reference sums it unrounded, which leaves dP - delta,
// where those nearly cancel (one vocabulary row, or one row with all of P),
// with the rounding error of gO alone (gh and gb then miss the fp32 formula by
// 2-7% in bf16 at V = 1, D = 300; 0.2% with the rounded sum).  Elsewhere the two
// sums agree to that rounding.
template <class T>
__global__ __launch_bounds__(256) void bwd_delta_kernel(const float* __restrict__ O, const float* __restrict__ gO,
                                                        const float* __restrict__ glse, int N, int D,
                                                        float* __restrict__ delta, int* __restrict__ flag) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  float s = 0.f;
  bool nz = false;
  for (int k = 0; k < D; ++k) {
    const float g = gO[(int64_t)n * D + k];
    s += O[(int64_t)n * D + k] * to_float(from_float<T>(g));
    nz |= g != 0.f;
  }
  s -= glse[n];
  delta[n] = s;
  flag[n] = nz || glse[n] != 0.f || s != 0.f;  // NaN != 0
}

// Order-preserving compaction of the active tokens: idx[q] = token of
// position q, inv[n] = position of token n or -1, n_act[0] = count.  One
// workgroup; each thread scans IT consecutive tokens per round.
__global__ __launch_bounds__(1024) void bwd_compact_kernel(const int* __restrict__ flag, int N, int* __restrict__ idx,
                                                           int* __restrict__ inv, int* __restrict__ n_act) {
  constexpr int IT = 16;
  __shared__ int wsum[16];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  int carry = 0;
  for (int base = 0; base < N; base += 1024 * IT) {
    const int n0 = base + t * IT;
    int f[IT];
    int cnt = 0;
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      f[i] = n0 + i < N ? flag[n0 + i] : 0;
      cnt += f[i];
    }
    int x = cnt;  // inclusive scan over the wave
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(x, o);
      if (lane >= o) x += y;
    }
    if (lane == 63) wsum[w] = x;
    __syncthreads();
    int before = 0, total = 0;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      before += j < w ? wsum[j] : 0;
      total += wsum[j];
    }
    int q = carry + before + x - cnt;
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int n = n0 + i;
      if (n < N) {
        inv[n] = f[i] ? q : -1;
        if (f[i]) idx[q++] = n;
      }
    }
    carry += total;
    __syncthreads();  // wsum is rewritten next round
  }
  if (t == 0) n_act[0] = carry;
}

// The token-side operands of the scores kernel over positions: gO rounded to
// the compute dtype (swvr/chunked.py:115) as [N_pad][DP] (zero padded), the
// same values transposed per token block as [N_pad / BM][DP][BM] with the
// positions of a block in pe_row order (the A operand of dE^T = gO^T P), and
// [lse | delta] as 2 x N_pad floats (lse = +inf on padding: P = 0 there).
template <class T>
__global__ __launch_bounds__(256) void bwd_pack_kernel(const float* __restrict__ gO, const float* __restrict__ lse,
                                                       const float* __restrict__ delta, const int* __restrict__ idx,
                                                       const int* __restrict__ n_act, int D, int N_pad, int DP, int BM,
                                                       T* __restrict__ gOp, T* __restrict__ gOt,
                                                       float* __restrict__ lsed) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= (int64_t)N_pad * DP) return;
  const int na = n_act[0];
  const int q = (int)(e / DP), d = (int)(e % DP);
  const int n = q < na ? idx[q] : -1;
  gOp[e] = (n >= 0 && d < D) ? from_float<T>(gO[(int64_t)n * D + d]) : (T)0.f;
  {
    const int64_t blk = e / ((int64_t)DP * BM);
    const int rem = (int)(e - blk * DP * BM);
    const int dt = rem / BM;
    const int qt = (int)(blk * BM) + pe_row(rem % BM);
    const int nt = qt < na ? idx[qt] : -1;
    gOt[e] = (nt >= 0 && dt < D) ? from_float<T>(gO[(int64_t)nt * D + dt]) : (T)0.f;
  }
  if (d == 0) {
    lsed[q] = n >= 0 ? lse[n] : kPosInf;
    lsed[N_pad + q] = n >= 0 ? delta[n] : 0.f;
  }
}

// h rows of the active tokens in position order, [N_pad][K] (zeros past
// n_act), 16 bytes of T per thread; h may be fp32 for a 2-byte T (rounded here).
template <class Src, class T>
__global__ __launch_bounds__(256) void bwd_gather_rows_kernel(const Src* __restrict__ h, int64_t ldh,
                                                              const int* __restrict__ idx,
                                                              const int* __restrict__ n_act, int N_pad, int K,
                                                              T* __restrict__ hc) {
  constexpr int CE = 16 / (int)sizeof(T);
  const int cpr = K / CE;
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= (int64_t)N_pad * cpr) return;
  const int q = (int)(e / cpr), c = (int)(e % cpr);
  const int n = q < n_act[0] ? idx[q] : -1;
  uint4 v = make_uint4(0, 0, 0, 0);
  if (n >= 0) v = load_chunk<Src, T>(h + (int64_t)n * ldh + (int64_t)c * CE);
  *reinterpret_cast<uint4*>(hc + (int64_t)q * K + (int64_t)c * CE) = v;
}

// gh from the fp32 accumulator over positions: row n = dh_acc row inv[n], or
// zero for an inactive token.  4 values per thread.
__global__ __launch_bounds__(256) void bwd_expand_kernel(const float* __restrict__ dh_acc, const int* __restrict__ inv,
                                                         int N, int K, void* __restrict__ gh, int gh_dtype) {
  const int cpr = K / 4;
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= (int64_t)N * cpr) return;
  const int n = (int)(e / cpr), c = (int)(e % cpr);
  const int q = inv[n];
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
  if (q >= 0) v = *reinterpret_cast<const float4*>(dh_acc + (int64_t)q * K + (int64_t)c * 4);
  const int64_t o = (int64_t)n * K + (int64_t)c * 4;
  if (gh_dtype == kBF16) {
    bf16_t* g = static_cast<bf16_t*>(gh) + o;
    g[0] = (bf16_t)v.x; g[1] = (bf16_t)v.y; g[2] = (bf16_t)v.z; g[3] = (bf16_t)v.w;
  } else if (gh_dtype == kF16) {
    f16_t* g = static_cast<f16_t*>(gh) + o;
    g[0] = (f16_t)v.x; g[1] = (f16_t)v.y; g[2] = (f16_t)v.z; g[3] = (f16_t)v.w;
  } else {
    *reinterpret_cast<float4*>(static_cast<float*>(gh) + o) = v;
  }
}

// ---------------------------------------------------------------- scores
struct ScoresParams {
  const void* hp;       // h packed in its tiles' LDS image (pack_rows_tiled_kernel)
  const void* Wp;       // the chunk's W rows packed the same way (its row 0 is row v0 of W)
  int hS;               // reduction slices of both
  const void* Ep;       // packed E [V_pad][DP]
  const float* biasp;   // packed bias [V_pad]
  const float* multp;   // e4m3 scores: logit_scale * h_scale * w_scale[v], [V_pad]; else null
  float scale;
  int N, K;
  const void* gOp;      // packed gO [N_pad][DP]
  const void* gOt;      // packed gO^T per token block [N_pad / BM][DP][BM], pe_row order
  const float* lsed;    // [lse | delta], 2 x N_pad
  int N_pad;
  int v0, cv;           // chunk start and rows
  int C;                // chunk stride of the partials (multiple of BV)
  int n_tb, G, n_vtc;
  void* stage;          // dS in the compute dtype, tiled (stage_off)
  void* pstage;         // P in the compute dtype, same layout (wide kernel: dE^T = gO^T P in the GEMM launch)
  int n_tb32;           // N_pad / 32: 32-token blocks of the stage
  float* part_dE;       // [G][DP][C]
  float* part_db;       // [G][C]
  int need_stage, need_dE, need_db;
  const int* n_act;     // active positions (device)
  int DP;               // padded embedding width (wide kernel: D-slices of gO and E)
};

// ---------------------------------------------------------------- dS stage layout
// The stage holds dS in 32 x 32 blocks, [C / 32][N_pad / 32][32 vocabulary
// rows][32 positions], each block contiguous (2 KB in bf16).  Position p of a
// block holds token stage_tok(p) of its 32 tokens: the order in which a lane
// of an MFMA accumulator holds tokens (register 4g + i of lane half hi is
// token 8g + 4hi + i), so a lane stores its 16 values as one run and a wave
// one whole block.  The gradient GEMMs reduce over positions (dW, with the
// matching rows of h) or produce rows in position order (dh, written back to
// their tokens).
__host__ __device__ __forceinline__ int stage_tok(int p) { return 8 * ((p & 15) >> 2) + 4 * (p >> 4) + (p & 3); }
// Element offset of (chunk-local vocabulary row v, position q).
__host__ __device__ __forceinline__ int64_t stage_off(int v, int q, int n_tb32) {
  return ((int64_t)(v >> 5) * n_tb32 + (q >> 5)) * 1024 + (v & 31) * 32 + (q & 31);
}

// One 32 x 32 accumulator block of dS (lane column: vocabulary row vc,
// registers: the block's 32 tokens from tok0) into the stage.
template <class T>
__device__ __forceinline__ void store_ds_block(const f32x16_t& ds, void* stage, int n_tb32, int vc, int tok0,
                                               int lane = lane_id()) {
  // Non-temporal stores: the stage is read back by the next launch, not by
  // this one, so its lines need not displace the operand slices in L2.
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  u32x4* dst = reinterpret_cast<u32x4*>(static_cast<T*>(stage) + stage_off(vc, tok0, n_tb32) + (lane >> 5) * 16);
  if constexpr (sizeof(T) == 2) {
    T q[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) q[r] = from_float<T>(ds[r]);
    u32x4 u[2];
    __builtin_memcpy(u, q, 32);
    __builtin_nontemporal_store(u[0], dst);
    __builtin_nontemporal_store(u[1], dst + 1);
  } else {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const u32x4 u = {__float_as_uint(ds[4 * g]), __float_as_uint(ds[4 * g + 1]), __float_as_uint(ds[4 * g + 2]),
                       __float_as_uint(ds[4 * g + 3])};
      __builtin_nontemporal_store(u, dst + g);
    }
  }
}

// Tile shape of the scores kernel per (dtype, padded D): BM tokens x BV
// vocabulary rows per workgroup of WT x WV waves (two waves per SIMD for
// bf16 / f16).  dE^T (DP x BV/WV per wave) and the score block share the
// register file; the stage ring, E, and the gO tile share LDS.
template <class T, int DP>
struct ScoresTile {
  static constexpr bool wide = sizeof(T) == 2;
  static constexpr int BM = wide ? (DP <= 128 ? 128 : 64) : 64;
  static constexpr int BV = wide ? (DP <= 64 ? 256 : 128) : 128;
  static constexpr int WT = wide && DP == 128 ? 2 : 1;
  static constexpr int WV = 4;
  static constexpr int NT = 64 * WT * WV;
  // LDS: the K-slice ring plus E [BV][DP], gO [BM][DP], gO^T [DP][BM], bias
  // and LSE / delta; the ring is as deep as the 160 KB allow (at most 4).
  static constexpr int SIDE = (BV + 2 * BM) * DP * (int)sizeof(T) + BV * 4 + 2 * BM * 4;
  static constexpr int SB = (BM + BV) * 64;
  static constexpr int NS = SIDE + 4 * SB <= 160 * 1024 ? 4 : SIDE + 3 * SB <= 160 * 1024 ? 3 : 2;
};

// One workgroup: BV vocabulary rows of the chunk x one group of token
// blocks.  Each wave owns BV/WV vocabulary rows and BM/WT tokens of every
// block, so dE / db of its rows accumulate in its registers for the whole
// group (one partial per token-wave row).  Scores use the S layout (A = h
// rows, B = W rows): a lane holds one vocabulary column and the registers
// hold tokens, which is the B-operand layout P needs for dE^T = gO^T P.
// F8: h and W packed from e4m3 bytes (read as bf16 pairs); the k64 e4m3
// reduction recomputes the scores the e4m3 forward computed.
template <class T, int DP, bool F8 = false>
__global__ __launch_bounds__((ScoresTile<T, DP>::NT)) void bwd_scores_kernel(ScoresParams p) {
  typedef ScoresTile<T, DP> C;
  typedef typename Vec8<T>::type V8;
  constexpr int kBK = SliceK<T>::value;
  constexpr int BM = C::BM, BV = C::BV, NT = C::NT;
  constexpr int WTR = BM / C::WT, WVR = BV / C::WV;  // rows per wave
  typedef PackedKLoader<T, BM, kBK, NT> TA;  // h rows of the token block (packed)
  typedef PackedKLoader<T, BV, kBK, NT> TB;  // W rows of the vocabulary tile (packed)
  typedef KTile<T, BV, DP, NT> TE;   // E tile
  typedef KTile<T, BM, DP, NT> TG;   // gO tile
  typedef KTile<T, DP, BM, NT> TGT;  // gO^T tile, tokens in pe_row order
  constexpr int SB = TA::BYTES + TB::BYTES;
  static_assert(SB == C::SB, "stage size");
  constexpr int L = TA::NI_MIN + TB::NI_MIN;  // conservative for partial tiles
  constexpr int FT = WTR / 32, FV = WVR / 32;
  constexpr int DB = DP / 32, DK = DP / 16;

  constexpr int NS = C::NS;
  __shared__ __attribute__((aligned(1024))) char smem[NS * SB + TE::BYTES + TG::BYTES + TGT::BYTES + BV * 4 + 2 * BM * 4];
  char* const sE = smem + NS * SB;
  char* const sG = sE + TE::BYTES;
  char* const sGt = sG + TG::BYTES;
  float* const sBias = reinterpret_cast<float*>(sGt + TGT::BYTES);
  float* const sLse = sBias + BV;
  float* const sDelta = sLse + BM;

  const int lane = lane_id(), w = wave_id();
  const int wt = w / C::WV, wv = w % C::WV;
  const int t = xcd_swizzle(blockIdx.x, p.n_vtc * p.G);
  const int vt = t / p.G, g = t % p.G;
  const int vl0 = vt * BV;      // first chunk-local row of this tile
  const int vg0 = p.v0 + vl0;   // its global row
  const int rows = p.cv - vl0;  // valid rows of this tile (may exceed BV)
  // token blocks of the active positions only, split evenly over the groups
  const int n_tb_act = min(p.n_tb, (p.n_act[0] + BM - 1) / BM);
  const int tb_begin = (int)((int64_t)g * n_tb_act / p.G);
  const int tb_end = (int)((int64_t)(g + 1) * n_tb_act / p.G);

  // E and bias of the vocabulary tile: once per workgroup, ahead of the stages
  const uint32_t lds0 = lds_addr(smem);
  const uint32_t ldsE = lds0 + NS * SB, ldsG = ldsE + TE::BYTES, ldsGt = ldsG + TG::BYTES;
  const uint32_t ldsB = ldsGt + TGT::BYTES;
  const uint32_t ldsL = ldsB + BV * 4;
  {
    TE te;
    te.setup(static_cast<const T*>(p.Ep) + (int64_t)vg0 * DP, DP, BV, DP);
    te.issue(ldsE, 0);
    if ((int)threadIdx.x * 16 < BV * 4) dma_batch1(make_rsrc(p.biasp + vg0), (uint32_t)threadIdx.x * 16, ldsB + w * 1024);
  }

  f32x16_t deacc[DB][FV];
  float dbacc[FV];
#pragma unroll
  for (int fv = 0; fv < FV; ++fv) {
    dbacc[fv] = 0.f;
#pragma unroll
    for (int db = 0; db < DB; ++db) deacc[db][fv] = zero16();
  }

  const int nk = max(1, (p.K + kBK - 1) / kBK);  // K = 0: one all-zero slice (bias-only scores)
  const int n_blocks = tb_end - tb_begin;
  TA ta;
  ta.setup(p.hp, tb_begin * BM, p.hS);
  TB tw;
  tw.setup(p.Wp, vl0, p.hS);
  // issue cursor: the next stage to load (NS - 1 ahead of the compute)
  int is_blk = 0, is_kt = 0, is_slot = 0;
  auto issue_next = [&]() {
    if (is_blk >= n_blocks) return;
    if (is_kt == 0) {
      const int n0 = (tb_begin + is_blk) * BM;
      ta.rebase(n0);
    }
    const uint32_t st = lds0 + is_slot * SB;
    ta.issue(st, is_kt * kBK);
    tw.issue(st + TA::BYTES, is_kt * kBK);
    if (++is_kt == nk) {
      is_kt = 0;
      ++is_blk;
    }
    is_slot = is_slot == NS - 1 ? 0 : is_slot + 1;
  };
#pragma unroll
  for (int s = 0; s < NS - 1; ++s) issue_next();

  f32x16_t sacc[FT][FV];
  Ring<NS> ring{NS - 1, n_blocks * nk};  // the first publish_next() moves to stage 0, slot 0
  for (int blk = 0; blk < n_blocks; ++blk) {
    const int n0 = (tb_begin + blk) * BM;
    // first stage of the block; every wave has also finished the previous
    // block's epilogue, so the gO / LSE / delta tiles can be replaced
    ring.template publish_next<L>();
    {
      TG tg;
      tg.setup(static_cast<const T*>(p.gOp) + (int64_t)n0 * DP, DP, BM, DP);
      tg.issue(ldsG, 0);
      TGT tgt;
      tgt.setup(static_cast<const T*>(p.gOt) + (int64_t)n0 * DP, BM, DP, BM);
      tgt.issue(ldsGt, 0);
      const int c = threadIdx.x;  // BM/4 chunks of LSE, then BM/4 of delta
      if (c < BM / 2) {
        const uint32_t off = c < BM / 4 ? (uint32_t)(n0 + 4 * c) * 4 : (uint32_t)(p.N_pad + n0 + 4 * (c - BM / 4)) * 4;
        dma_batch1(make_rsrc(p.lsed), off, ldsL + w * 1024);
      }
    }
#pragma unroll
    for (int ft = 0; ft < FT; ++ft)
#pragma unroll
      for (int fv = 0; fv < FV; ++fv) sacc[ft][fv] = zero16();
    if constexpr (F8)
      tile_reduce_f8<L, false>(sacc, ta, tw, smem, SB, ring, nk, wt * WTR, wv * WVR, issue_next);
    else
      tile_reduce<T, kBK, L>(sacc, ta, tw, smem, SB, ring, nk, wt * WTR, wv * WVR, issue_next);
    if (nk <= NS) {
      // short reduction: the side loads (gO / LSE / delta, and E / bias of
      // the first block) may still be in flight
      wait_vmcnt<0>();
      stage_barrier();
    }

    TG tgl;  // layout only
    TE tel;
#pragma unroll
    for (int fv = 0; fv < FV; ++fv) {
      const int vl = wv * WVR + fv * 32 + (lane & 31);  // tile-local row of this lane
      const float bvv = vl < rows ? sBias[vl] : kNegInf;
      const float mvv = F8 ? (vl < rows ? p.multp[vg0 + vl] : 0.f) : p.scale;
#pragma unroll
      for (int ft = 0; ft < FT; ++ft) {
        // LDS bases recomputed per block (see opaque_zero)
        const int oz = opaque_zero();
        const char* sGe = sG + oz;
        const char* sGte = sGt + oz;
        const char* sEe = sE + oz;
        const float* sLe = sLse + oz;
        const float* sDe = sDelta + oz;
        const int tr0 = wt * WTR + ft * 32;  // first token of the block
        // dP block = gO[tokens] E[rows]^T over D
        f32x16_t dp = zero16();
#pragma unroll
        for (int kd = 0; kd < DK; ++kd)
          mfma_k16(dp, read_op(tgl, sGe, tr0 + (lane & 31), kd), read_op(tel, sEe, vl, kd));
        float dbs = 0.f;
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          // registers 4g..4g+3 hold tokens 8g + 4(lane/32) + 0..3 of the block
          const int tl = tr0 + 8 * g4 + (lane >> 5) * 4;
          const float4 l4 = *reinterpret_cast<const float4*>(sLe + tl);
          const float4 d4 = *reinterpret_cast<const float4*>(sDe + tl);
          const float lv[4] = {l4.x, l4.y, l4.z, l4.w}, dv[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = 4 * g4 + i;
            const float pv = fast_exp(fmaf(sacc[ft][fv][r], mvv, bvv) - lv[i]);
            const float ds = pv * (dp[r] - dv[i]);
            dbs += ds;
            sacc[ft][fv][r] = pv;
            dp[r] = ds;  // the gradient GEMMs apply the scale (swvr/chunked.py:143-144)
          }
        }
        dbacc[fv] += dbs;
        if (p.need_stage) store_ds_block<T>(dp, p.stage, p.n_tb32, vl0 + vl, n0 + tr0);
        if (p.need_dE) {
          // dE^T[d][v] += gO^T[d][tok] P[tok][v]; registers 8c..8c+7 hold
          // tokens 16c + 8(t/4) + 4(lane/32) + t%4, stored contiguously in
          // the gO^T tile (pe_row order): one read per operand
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            V8 bv;
#pragma unroll
            for (int tt = 0; tt < 8; ++tt) bv[tt] = from_float<T>(sacc[ft][fv][8 * c + tt]);
            const int p0 = tr0 + 8 * (2 * c + (lane >> 5));
#pragma unroll
            for (int db = 0; db < DB; ++db) {
              const int d = db * 32 + (lane & 31);
              V8 av;
              if constexpr (sizeof(T) == 2) {
                av = *reinterpret_cast<const V8*>(sGte + TGT::elem(d, p0));
              } else {
                const float4 lo = *reinterpret_cast<const float4*>(sGte + TGT::elem(d, p0));
                const float4 hi = *reinterpret_cast<const float4*>(sGte + TGT::elem(d, p0 + 4));
                av[0] = lo.x; av[1] = lo.y; av[2] = lo.z; av[3] = lo.w;
                av[4] = hi.x; av[5] = hi.y; av[6] = hi.z; av[7] = hi.w;
              }
              mfma_k16(deacc[db][fv], av, bv);
            }
          }
        }
        sched_fence();
      }
    }
  }

  // partials of this wave's rows over its token share of the group
  const int gp = g * C::WT + wt;
#pragma unroll
  for (int fv = 0; fv < FV; ++fv) {
    const int vc = vl0 + wv * WVR + fv * 32 + (lane & 31);  // chunk-local row
    if (p.need_db) {
      const float s = wave_sum32(dbacc[fv]);
      if (lane < 32) p.part_db[(int64_t)gp * p.C + vc] = s;
    }
    if (p.need_dE) {
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int d = db * 32 + c_row(r, lane);
          p.part_dE[((int64_t)gp * DP + d) * p.C + vc] = deacc[db][fv][r];
        }
    }
  }
}

// ---------------------------------------------------------------- scores, narrow embeddings
// bf16 / f16 with DP <= 64: 256 tokens x 256 vocabulary rows per workgroup of
// 8 waves (2 token halves x 4 vocabulary quarters, 128 x 64 per wave, 0.75
// operand reads per MFMA).  The LDS is a 4-slot ring of 32 KB; per token block
// it carries the nk K-slices of h and W, then the side tiles of the epilogue:
// E [BV][DP], gO [BM][DP] and gO^T [DP][BM] (tokens in pe_row order).
//   DP = 64: three side stages; their slots stay pinned through the epilogue,
//   and the next block's slices catch up after it.
//   DP = 32: E (16 KB, the same for the workgroup's whole walk) is loaded once
//   into an LDS region of its own, and gO and gO^T (16 KB each) share one side
//   stage, so three slots stay free through the epilogue and the ring carries
//   the next block's first slices without a pause.
// The bias sits in registers, LSE / delta in a double-buffered LDS strip.
template <class T, int DP>
struct ScoresRingTile {
  static constexpr int BM = 256, BV = 256, WT = 2, WV = 4, NT = 64 * WT * WV, NS = 4;
};

template <class T, int DP, bool F8 = false>
__global__ __launch_bounds__(512) void bwd_scores_ring_kernel(ScoresParams p) {
  typedef ScoresRingTile<T, DP> C;
  typedef typename Vec8<T>::type V8;
  constexpr int kBK = SliceK<T>::value;
  constexpr int BM = C::BM, BV = C::BV, NT = C::NT, NS = C::NS;
  constexpr int WTR = BM / C::WT, WVR = BV / C::WV;  // rows per wave
  typedef PackedKLoader<T, BM, kBK, NT> TA;  // h rows of the token block (packed)
  typedef PackedKLoader<T, BV, kBK, NT> TB;  // W rows of the vocabulary tile (packed)
  typedef KTile<T, BV, DP, NT> TE;   // E tile
  typedef KTile<T, BM, DP, NT> TG;   // gO tile
  typedef KTile<T, DP, BM, NT> TGT;  // gO^T tile, tokens in pe_row order
  constexpr int SB = TA::BYTES + TB::BYTES;
  constexpr int L = TA::NI + TB::NI;  // loads per thread per stage, side stages padded to it
  static_assert(!TA::PARTIAL && !TB::PARTIAL && !TE::PARTIAL && !TG::PARTIAL && !TGT::PARTIAL, "whole loads");
  static_assert(TE::NI <= L && TG::NI <= L && TGT::NI <= L, "side tiles fit a slot");
  constexpr int FT = WTR / 32, FV = WVR / 32;
  constexpr int DB = DP / 32, DK = DP / 16;
  // E pinned in its own region, gO and gO^T in one side stage (see above)
  constexpr bool PIN_E = DP == 32 && !F8;
  static_assert(!PIN_E || (TG::BYTES + TGT::BYTES == SB && TG::NI + TGT::NI == L), "gO | gO^T fill one stage");
  constexpr int N_SIDE = PIN_E ? 1 : 3;  // side stages per token block

  __shared__ __attribute__((aligned(1024)))
  char smem[NS * SB + 2 * 2 * BM * 4 + (F8 ? BV * 8 : 0) + (PIN_E ? TE::BYTES : 0)];
  float* const sLD = reinterpret_cast<float*>(smem + NS * SB);  // [2 buffers][LSE BM | delta BM]
  // F8: (bias, score factor) of the tile's rows, read in the epilogue (two fewer registers per
  // row block than holding both); the bf16 kernel holds the bias in registers
  float2* const sBM = reinterpret_cast<float2*>(smem + NS * SB + 2 * 2 * BM * 4);
  // PIN_E: the workgroup's E tile
  char* const sEpin = smem + NS * SB + 2 * 2 * BM * 4;

  const int lane = lane_id(), w = wave_id();
  const int wt = w / C::WV, wv = w % C::WV;
  int vt, g;
  grouped_tile(blockIdx.x, p.n_vtc, p.G, &vt, &g);
  const int vl0 = vt * BV;      // first chunk-local row of this tile
  const int vg0 = p.v0 + vl0;   // its global row
  const int rows = p.cv - vl0;  // valid rows of this tile (may exceed BV)
  // token blocks of the active positions only, split evenly over the groups
  const int n_tb_act = min(p.n_tb, (p.n_act[0] + BM - 1) / BM);
  const int tb_begin = (int)((int64_t)g * n_tb_act / p.G);
  const int tb_end = (int)((int64_t)(g + 1) * n_tb_act / p.G);
  const int n_blocks = tb_end - tb_begin;

  // visible to every wave after the first stage's barrier, before any epilogue
  if constexpr (F8)
    for (int i = threadIdx.x; i < BV; i += NT)
      sBM[i] = make_float2(i < rows ? p.biasp[vg0 + i] : kNegInf, i < rows ? p.multp[vg0 + i] : 0.f);
  f32x16_t deacc[DB][FV];
  float dbacc[FV], bvv[FV];
#pragma unroll
  for (int fv = 0; fv < FV; ++fv) {
    dbacc[fv] = 0.f;
    const int vl = wv * WVR + fv * 32 + (lane & 31);
    if constexpr (!F8) bvv[fv] = vl < rows ? p.biasp[vg0 + vl] : kNegInf;
#pragma unroll
    for (int db = 0; db < DB; ++db) deacc[db][fv] = zero16();
  }

  const int nk = max(1, (p.K + kBK - 1) / kBK);  // K = 0: one all-zero slice (bias-only scores)
  const int per_blk = nk + N_SIDE;
  const int total = n_blocks * per_blk;
  const uint32_t lds0 = lds_addr(smem);
  const uint32_t ldsL = lds0 + NS * SB;
  TA ta;
  ta.setup(p.hp, tb_begin * BM, p.hS);
  TB tw;
  tw.setup(p.Wp, vl0, p.hS);
  const rsrc_t r_none = make_rsrc(nullptr);
  // issue cursor over the walk: stage `issued` is (block is_blk, sub-stage
  // is_sub) into slot is_slot; sub-stages 0..nk-1 are K-slices, nk, nk+1, nk+2
  // the E, gO and gO^T tiles
  int issued = 0, is_blk = 0, is_sub = 0, is_slot = 0;
  auto pad = [&](int n_real, uint32_t st) {  // zero-filling loads up to L per thread
#pragma unroll
    for (int i = n_real; i < L; ++i) dma_batch1(r_none, kOOB, st + i * NT * 16 + w * 1024);
  };
  auto issue_next = [&]() {
    if (issued >= total) return;
    const uint32_t st = lds0 + is_slot * SB;
    const int n0 = (tb_begin + is_blk) * BM;
    if (is_sub < nk) {
      if (is_sub == 0) {
        ta.rebase(n0);
        // LSE and delta of the block into strip (block & 1), ahead of its slices
        // (offsets recomputed per block, see opaque_zero)
        const int c = (int)threadIdx.x + opaque_zero();
        if (c < BM / 2) {
          const uint32_t off = c < BM / 4 ? (uint32_t)(n0 + 4 * c) * 4 : (uint32_t)(p.N_pad + n0 + 4 * (c - BM / 4)) * 4;
          dma_batch1(make_rsrc(p.lsed), off, ldsL + (is_blk & 1) * (2 * BM * 4) + w * 1024);
        }
      }
      ta.issue(st, is_sub * kBK);
      tw.issue(st + TA::BYTES, is_sub * kBK);
    } else if (PIN_E) {
      // gO in the stage's first half, gO^T in its second
      TG tg;
      tg.setup(static_cast<const T*>(p.gOp) + (int64_t)n0 * DP, DP, BM, DP, (int)threadIdx.x + opaque_zero());
      tg.issue(st, 0);
      TGT tgt;
      tgt.setup(static_cast<const T*>(p.gOt) + (int64_t)n0 * DP, BM, DP, BM, (int)threadIdx.x + opaque_zero());
      tgt.issue(st + TG::BYTES, 0);
    } else if (is_sub == nk) {
      TE te;
      // an opaque thread index: the load offsets are computed here, once per
      // block, instead of being hoisted out of the walk (registers)
      te.setup(static_cast<const T*>(p.Ep) + (int64_t)vg0 * DP, DP, BV, DP, (int)threadIdx.x + opaque_zero());
      te.issue(st, 0);
      pad(TE::NI, st);
    } else if (is_sub == nk + 1) {
      TG tg;
      tg.setup(static_cast<const T*>(p.gOp) + (int64_t)n0 * DP, DP, BM, DP, (int)threadIdx.x + opaque_zero());
      tg.issue(st, 0);
      pad(TG::NI, st);
    } else {
      TGT tgt;
      tgt.setup(static_cast<const T*>(p.gOt) + (int64_t)n0 * DP, BM, DP, BM, (int)threadIdx.x + opaque_zero());
      tgt.issue(st, 0);
      pad(TGT::NI, st);
    }
    ++issued;
    if (++is_sub == per_blk) {
      is_sub = 0;
      ++is_blk;
    }
    is_slot = is_slot == NS - 1 ? 0 : is_slot + 1;
  };
  if constexpr (PIN_E) {
    // the E tile, ahead of every stage: the first stage's wait covers it
    if (total > 0) {
      TE te;
      te.setup(static_cast<const T*>(p.Ep) + (int64_t)vg0 * DP, DP, BV, DP);
      te.issue(lds_addr(sEpin), 0);
    }
  }
#pragma unroll
  for (int s = 0; s < NS - 1; ++s) issue_next();

  f32x16_t sacc[FT][FV];
  CountedRing<NS> ring{NS - 1, -1, &issued};
  ring.template publish_next<L>();  // block 0, slice 0
  for (int blk = 0; blk < n_blocks; ++blk) {
    const int n0 = (tb_begin + blk) * BM;
    if (blk > 0) {
      // slice 0 of this block: every wave has finished the previous epilogue.
      // DP = 64: its three side slots are free: catch up to NS - 1 stages
      // ahead.  DP = 32: the ring stayed NS - 1 stages ahead through it.
      ring.template publish_next<L>();
      if constexpr (!PIN_E) {
        issue_next();
        issue_next();
      }
    }
#pragma unroll
    for (int ft = 0; ft < FT; ++ft)
#pragma unroll
      for (int fv = 0; fv < FV; ++fv) sacc[ft][fv] = zero16();
    if constexpr (F8)
      tile_reduce_f8<L, false>(sacc, ta, tw, smem, SB, ring, nk, wt * WTR, wv * WVR, issue_next);
    else
      tile_reduce<T, kBK, L>(sacc, ta, tw, smem, SB, ring, nk, wt * WTR, wv * WVR, issue_next);
    int slot_gt;
    if constexpr (PIN_E) {
      ring.template publish_next<L>();  // gO | gO^T
      issue_next();                     // the next block's slice 2 into the last slice's slot
      slot_gt = ring.slot;
    } else {
      ring.template publish_next<L>();  // E
      issue_next();                     // the next block's slice 0 into the last slice's slot
      ring.template publish_next<L>();  // gO
      ring.template publish_next<L>();  // gO^T
      slot_gt = ring.slot;
    }

    TG tgl;  // layout only
    TE tel;
    // dP block (fv, ft) = gO[tokens] E[rows]^T over D.  Every lane-dependent
    // offset in the epilogue derives from an opaque copy of the lane's row (see
    // opaque_zero), so it is recomputed per block: hoisted out of the block loop
    // the offsets would be spilled, and each reload from scratch waits (vmcnt in
    // order) for every store issued before it.  The side tiles sit in the three
    // slots before and at the current one (DP = 32: gO and gO^T in the current
    // slot, E in its own region).
    auto dp_block = [&](int fv, int ft) {
      const int ln = lane + opaque_zero();
      const int lr = ln & 31;
      const char* sGe = PIN_E ? smem + slot_gt * SB : smem + ((slot_gt + NS - 1) % NS) * SB;
      const char* sEe = PIN_E ? static_cast<const char*>(sEpin) : smem + ((slot_gt + NS - 2) % NS) * SB;
      f32x16_t d = zero16();
#pragma unroll
      for (int kd = 0; kd < DK; ++kd)
        mfma_k16(d, read_op(tgl, sGe, wt * WTR + ft * 32 + lr, kd, ln),
                 read_op(tel, sEe, wv * WVR + fv * 32 + lr, kd, ln));
      return d;
    };
    // software-pipelined by one block: the dP products of the next block run
    // on the matrix cores while this block's exponentials and stores run
    f32x16_t dp_next = dp_block(0, 0);
#pragma unroll
    for (int fv = 0; fv < FV; ++fv) {
#pragma unroll
      for (int ft = 0; ft < FT; ++ft) {
        f32x16_t dp = dp_next;
        constexpr int kBlocks = FV * FT;
        const int nb = fv * FT + ft + 1;
        if (nb < kBlocks) dp_next = dp_block(nb / FT, nb % FT);
        const int ln = lane + opaque_zero();
        const int lr = ln & 31;
        const int vl = wv * WVR + fv * 32 + lr;  // tile-local row of this lane
        const char* sGte = smem + slot_gt * SB + (PIN_E ? TG::BYTES : 0);
        const float* sLe = sLD + (blk & 1) * (2 * BM);
        const float* sDe = sLe + BM;
        const int tr0 = wt * WTR + ft * 32;  // first token of the block
        float dbs = 0.f;
        const float2 bm = F8 ? sBM[vl] : make_float2(bvv[fv], p.scale);  // this lane's row: bias, score factor
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          // registers 4g..4g+3 hold tokens 8g + 4(lane/32) + 0..3 of the block
          const int tl = tr0 + 8 * g4 + (ln >> 5) * 4;
          const float4 l4 = *reinterpret_cast<const float4*>(sLe + tl);
          const float4 d4 = *reinterpret_cast<const float4*>(sDe + tl);
          const float lv[4] = {l4.x, l4.y, l4.z, l4.w}, dv[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = 4 * g4 + i;
            const float pv = fast_exp(fmaf(sacc[ft][fv][r], bm.y, bm.x) - lv[i]);
            const float ds = pv * (dp[r] - dv[i]);
            dbs += ds;
            sacc[ft][fv][r] = pv;
            dp[r] = ds;  // the gradient GEMMs apply the scale (swvr/chunked.py:143-144)
          }
        }
        dbacc[fv] += dbs;
        if (p.need_stage) store_ds_block<T>(dp, p.stage, p.n_tb32, vl0 + vl, n0 + tr0, ln);
        if (p.need_dE) {
          // dE^T[d][v] += gO^T[d][tok] P[tok][v]; registers 8c..8c+7 hold
          // tokens 16c + 8(t/4) + 4(lane/32) + t%4, stored contiguously in
          // the gO^T tile (pe_row order): one read per operand
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            V8 bv;
#pragma unroll
            for (int tt = 0; tt < 8; ++tt) bv[tt] = from_float<T>(sacc[ft][fv][8 * c + tt]);
            const int p0 = tr0 + 8 * (2 * c + (ln >> 5));
#pragma unroll
            for (int db = 0; db < DB; ++db) {
              const V8 av = *reinterpret_cast<const V8*>(sGte + TGT::elem(db * 32 + lr, p0));
              mfma_k16(deacc[db][fv], av, bv);
            }
          }
        }
        sched_fence();
      }
    }
  }
  wait_vmcnt<0>();

  // partials of this wave's rows over its token share of the group (thread
  // offsets from an opaque thread index: computed here, not kept live through the walk)
  const int to = (int)threadIdx.x + opaque_zero();
  const int lo = to & 63, wo = to >> 6;
  const int gp = g * C::WT + wo / C::WV;
#pragma unroll
  for (int fv = 0; fv < FV; ++fv) {
    const int vc = vl0 + (wo % C::WV) * WVR + fv * 32 + (lo & 31);  // chunk-local row
    if (p.need_db) {
      const float s = wave_sum32(dbacc[fv]);
      if (lo < 32) p.part_db[(int64_t)gp * p.C + vc] = s;
    }
    if (p.need_dE) {
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int d = db * 32 + c_row(r, lo);
          p.part_dE[((int64_t)gp * DP + d) * p.C + vc] = deacc[db][fv][r];
        }
    }
  }
}

// ---------------------------------------------------------------- scores, wide embeddings
// bf16 / f16 with DP > 64 and fp32 with DP > 128 (DP any multiple of the
// slice width: 32 elements, 16 for fp32): 256 tokens (fp32: 128) x 256 vocabulary rows per
// workgroup of 8 waves (2 token halves x 4 vocabulary quarters: 128 x 64 each, 0.75 operand reads
// per MFMA; fp32 64 x 64).  Per token block the ring carries the nk K-slices of h and W (-> S),
// then the DP / 32 D-slices of gO and E (-> dP = gO E^T) once per 64 tokens of a wave's rows (a
// wave holds S for all its rows but dP for 64 of them: both whole would take 256 registers), all
// as uniform 32 KB stages (fp32: 24 KB), so no side tile is pinned in LDS and the next block's
// slices keep streaming through the epilogue.  The epilogue stages dS and P in the compute dtype (P
// rounded as the reference rounds it for dE, swvr/triton_kernels.py:113);
// dE^T = gO^T P is a product of the gradient GEMM launch over all active
// positions, so no dE accumulator lives in registers; db is a per-wave
// register partial.  LSE / delta sit in a double-buffered LDS strip, the bias
// in registers.
template <class T>
struct ScoresWideTile {
  static constexpr int BM = sizeof(T) == 2 ? 256 : 128, BV = 256, WT = 2, WV = 4, NT = 64 * WT * WV, NS = 4;
};

template <class T>
__global__ __launch_bounds__(512) void bwd_scores_wide_kernel(ScoresParams p) {
  typedef ScoresWideTile<T> C;
  constexpr int kBK = SliceK<T>::value;
  constexpr int BM = C::BM, BV = C::BV, NT = C::NT, NS = C::NS;
  constexpr int WTR = BM / C::WT, WVR = BV / C::WV;  // rows per wave
  typedef PackedKLoader<T, BM, kBK, NT> TA;  // h rows of the token block (packed)
  typedef PackedKLoader<T, BV, kBK, NT> TB;  // W rows of the vocabulary tile (packed)
  typedef KTile<T, BM, kBK, NT> TG;          // gO rows of the token block, one D-slice
  typedef KTile<T, BV, kBK, NT> TE;          // E rows of the vocabulary tile, one D-slice
  static_assert(TG::BYTES == TA::BYTES && TE::BYTES == TB::BYTES && TG::NI == TA::NI && TE::NI == TB::NI,
                "K- and D-stages load the same bytes");
  static_assert(!TA::PARTIAL && !TB::PARTIAL, "whole loads");
  constexpr int SB = TA::BYTES + TB::BYTES;
  constexpr int L = TA::NI + TB::NI;  // loads per thread per stage
  constexpr int FT = WTR / 32, FV = WVR / 32;
  constexpr int NPASS = FT / 2;  // dP passes per token block, 64 of a wave's rows each
  const int DP = p.DP;        // a multiple of the slice width kBK
  const int ND = DP / kBK;    // D-slices per dP pass

  __shared__ __attribute__((aligned(1024))) char smem[NS * SB + 2 * 2 * BM * 4];
  const float* const sLD = reinterpret_cast<const float*>(smem + NS * SB);  // [2 buffers][LSE BM | delta BM]

  const int lane = lane_id(), w = wave_id();
  const int wt = w / C::WV, wv = w % C::WV;
  int vt, g;
  grouped_tile(blockIdx.x, p.n_vtc, p.G, &vt, &g);
  const int vl0 = vt * BV;      // first chunk-local row of this tile
  const int vg0 = p.v0 + vl0;   // its global row
  const int rows = p.cv - vl0;  // valid rows of this tile (may exceed BV)
  // token blocks of the active positions only, split evenly over the groups
  const int n_tb_act = min(p.n_tb, (p.n_act[0] + BM - 1) / BM);
  const int tb_begin = (int)((int64_t)g * n_tb_act / p.G);
  const int tb_end = (int)((int64_t)(g + 1) * n_tb_act / p.G);
  const int n_blocks = tb_end - tb_begin;

  float dbacc[FV], bvv[FV];
#pragma unroll
  for (int fv = 0; fv < FV; ++fv) {
    dbacc[fv] = 0.f;
    const int vl = wv * WVR + fv * 32 + (lane & 31);
    bvv[fv] = vl < rows ? p.biasp[vg0 + vl] : kNegInf;
  }

  const int nk = max(1, (p.K + kBK - 1) / kBK);  // K = 0: one all-zero slice (bias-only scores)
  const int per_blk = nk + NPASS * ND;
  const int total = n_blocks * per_blk;
  const uint32_t lds0 = lds_addr(smem);
  const uint32_t ldsL = lds0 + NS * SB;
  TA ta;
  ta.setup(p.hp, tb_begin * BM, p.hS);
  TB tw;
  tw.setup(p.Wp, vl0, p.hS);
  const T* const gOp = static_cast<const T*>(p.gOp);
  TG tg;
  tg.setup(gOp + (int64_t)tb_begin * BM * DP, DP, BM, DP);
  TE te;
  te.setup(static_cast<const T*>(p.Ep) + (int64_t)vg0 * DP, DP, BV, DP);
  // issue cursor over the walk: stage `issued` is (block is_blk, sub-stage
  // is_sub) into slot is_slot; sub-stages 0..nk-1 are K-slices, nk.. the D-slices
  // of each dP pass in turn
  int issued = 0, is_blk = 0, is_sub = 0, is_slot = 0;
  auto issue_next = [&]() {
    if (issued >= total) return;
    const uint32_t st = lds0 + is_slot * SB;
    const int n0 = (tb_begin + is_blk) * BM;
    if (is_sub < nk) {
      if (is_sub == 0) {
        ta.rebase(n0);
        // LSE and delta of the block into strip (block & 1), ahead of its slices
        const int c = (int)threadIdx.x + opaque_zero();
        if (c < BM / 2) {
          const uint32_t off = c < BM / 4 ? (uint32_t)(n0 + 4 * c) * 4 : (uint32_t)(p.N_pad + n0 + 4 * (c - BM / 4)) * 4;
          dma_batch1(make_rsrc(p.lsed), off, ldsL + (is_blk & 1) * (2 * BM * 4) + w * 1024);
        }
      }
      ta.issue(st, is_sub * kBK);
      tw.issue(st + TA::BYTES, is_sub * kBK);
    } else {
      if (is_sub == nk) tg.base = reinterpret_cast<const char*>(gOp + (int64_t)n0 * DP);
      const int d0 = ((is_sub - nk) % ND) * kBK;
      tg.issue(st, d0);
      te.issue(st + TA::BYTES, d0);
    }
    ++issued;
    if (++is_sub == per_blk) {
      is_sub = 0;
      ++is_blk;
    }
    is_slot = is_slot == NS - 1 ? 0 : is_slot + 1;
  };
#pragma unroll
  for (int s = 0; s < NS - 1; ++s) issue_next();

  f32x16_t sacc[FT][FV], dacc[2][FV];
  Ring<NS> ring{NS - 1, total};  // the first publish_next() moves to stage 0, slot 0
  for (int blk = 0; blk < n_blocks; ++blk) {
    const int n0 = (tb_begin + blk) * BM;
    // slice 0 of the block: every wave has also finished the previous block's
    // epilogue (its LSE / delta strip is free again)
    ring.template publish_next<L>();
#pragma unroll
    for (int ft = 0; ft < FT; ++ft)
#pragma unroll
      for (int fv = 0; fv < FV; ++fv) sacc[ft][fv] = zero16();
    tile_reduce<T, kBK, L>(sacc, ta, tw, smem, SB, ring, nk, wt * WTR, wv * WVR, issue_next);

    const float* sLe = sLD + (blk & 1) * (2 * BM);
    const float* sDe = sLe + BM;
#pragma unroll
    for (int ps = 0; ps < NPASS; ++ps) {
      ring.template publish_next<L>();  // D-slice 0 of this pass
#pragma unroll
      for (int f2 = 0; f2 < 2; ++f2)
#pragma unroll
        for (int fv = 0; fv < FV; ++fv) dacc[f2][fv] = zero16();
      tile_reduce<T, kBK, L>(dacc, tg, te, smem, SB, ring, ND, wt * WTR + ps * 64, wv * WVR, issue_next);
#pragma unroll
      for (int fv = 0; fv < FV; ++fv) {
#pragma unroll
        for (int f2 = 0; f2 < 2; ++f2) {
          const int ft = 2 * ps + f2;
          const int ln = lane + opaque_zero();  // offsets recomputed per block (see opaque_zero)
          const int vl = wv * WVR + fv * 32 + (ln & 31);  // tile-local row of this lane
          const int tr0 = wt * WTR + ft * 32;             // first token of the block
          float dbs = 0.f;
#pragma unroll
          for (int g4 = 0; g4 < 4; ++g4) {
            // registers 4g..4g+3 hold tokens 8g + 4(lane/32) + 0..3 of the block
            const int tl = tr0 + 8 * g4 + (ln >> 5) * 4;
            const float4 l4 = *reinterpret_cast<const float4*>(sLe + tl);
            const float4 d4 = *reinterpret_cast<const float4*>(sDe + tl);
            const float lv[4] = {l4.x, l4.y, l4.z, l4.w}, dv[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int r = 4 * g4 + i;
              const float pv = fast_exp(fmaf(sacc[ft][fv][r], p.scale, bvv[fv]) - lv[i]);
              const float ds = pv * (dacc[f2][fv][r] - dv[i]);
              dbs += ds;
              sacc[ft][fv][r] = pv;
              dacc[f2][fv][r] = ds;  // the gradient GEMMs apply the scale (swvr/chunked.py:143-144)
            }
          }
          dbacc[fv] += dbs;
          if (p.need_stage) store_ds_block<T>(dacc[f2][fv], p.stage, p.n_tb32, vl0 + vl, n0 + tr0, ln);
          if (p.need_dE) store_ds_block<T>(sacc[ft][fv], p.pstage, p.n_tb32, vl0 + vl, n0 + tr0, ln);
          sched_fence();
        }
      }
    }
  }
  wait_vmcnt<0>();

  if (p.need_db) {
    const int gp = g * C::WT + wt;
#pragma unroll
    for (int fv = 0; fv < FV; ++fv) {
      const int vc = vl0 + wv * WVR + fv * 32 + (lane & 31);  // chunk-local row
      const float s = wave_sum32(dbacc[fv]);
      if (lane < 32) p.part_db[(int64_t)gp * p.C + vc] = s;
    }
  }
}

// ---------------------------------------------------------------- dE / db
// gE and gb rows of a chunk from their partials, summed over the partials in a
// fixed order (g ascending).  G_de: partials of dE ([G_de][DP][C]; 1 when the
// gradient GEMM formed dE^T whole), G: partials of db ([G][C]).  One workgroup
// of NT threads per tile of NT / 8 chunk rows x kRedD columns (kRedV for the
// 256-thread kernel): the partial reads run along the rows (consecutive v, as
// the partials store them), the sums pass through LDS, and gE is written along
// its rows (consecutive d), so both sides coalesce.  The workgroups of column
// tile 0 also write gb of their rows.
constexpr int kRedV = 32, kRedD = 16;

// sum_{g < n} p[g * stride] in order g = 0, 1, ...; the loads go out in batches of 8
// ahead of their adds, so a long sum waits for memory once per batch, not once per term.
__device__ __forceinline__ float ordered_sum(const float* __restrict__ p, int64_t stride, int n) {
  float s = 0.f;
  for (int g0 = 0; g0 < n; g0 += 8) {
    float x[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) x[u] = g0 + u < n ? p[(int64_t)(g0 + u) * stride] : 0.f;
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (g0 + u < n) s += x[u];
  }
  return s;
}

// The dE / db rows of the tile at chunk row vb, column db0; tile: [NT / 8][kRedD + 1] floats of LDS.
template <int NT>
__device__ __forceinline__ void reduce_tile(float (*tile)[kRedD + 1], const float* __restrict__ part_dE,
                                            const float* __restrict__ part_db, int G_de, int G, int C, int DP,
                                            int v0, int cv, int D, void* gE, int gE_dtype, float* gb, int vb,
                                            int db0) {
  constexpr int RV = NT / 8;
  const int t = threadIdx.x;
  if (gE) {
#pragma unroll
    for (int j = 0; j < RV * kRedD / NT; ++j) {
      const int i = j * NT + t;
      const int dl = i / RV, vl = i % RV;  // consecutive threads: consecutive rows
      const int v = vb + vl, d = db0 + dl;
      tile[vl][dl] = v < cv && d < D ? ordered_sum(part_dE + (int64_t)d * C + v, (int64_t)DP * C, G_de) : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < RV * kRedD / NT; ++j) {
      const int i = j * NT + t;
      const int vl = i / kRedD, dl = i % kRedD;  // consecutive threads: consecutive columns
      const int v = vb + vl, d = db0 + dl;
      if (v < cv && d < D) store_as(gE, (int64_t)(v0 + v) * D + d, gE_dtype, tile[vl][dl]);
    }
  }
  if (gb && db0 == 0 && t < RV) {
    const int v = vb + t;
    if (v < cv) gb[v0 + v] = ordered_sum(part_db + v, C, G);
  }
}

// ---------------------------------------------------------------- GEMMs
struct GemmParams {
  const void* stage;  // tiled dS (stage_off)
  int n_tb32;
  int64_t N_pad;
  const void* h;   // h rows in position order
  int64_t ldh;
  const void* W;   // W rows from row w_row0 on, row-major
  int64_t ldw;
  int w_row0;
  int N, K;
  int v0, cv;
  int n_n;         // tiles along K
  int n_dw, n_dh;  // tile counts (0 when that gradient is not needed)
  void* gW;
  int gW_dtype;
  float* dh_acc;   // dh over positions, fp32
  int dh_first;
  float scale;     // logit scale: the stage holds dS, the products are scale * stage^T h and scale * stage W
  const int* n_act;  // active positions (device): the reduction length of dW, the rows of dh
  // dE^T = gO^T P over positions (wide scores kernel): n_de tiles, n_de_n of them along the chunk,
  // each the reduction over one of de_split equal runs of the positions
  int n_de, n_de_n, de_split;
  const void* pstage;  // P, tiled like the dS stage
  const void* gOp;     // gO over positions [N_pad][DP]
  int DP;
  float* part_dE;      // output dE^T partials [de_split][DP][C], fp32 (the scores kernels' dE partials when n_red > 0)
  int C;
  // the chunk's dE / db reduction (reduce_tile), as n_red workgroups after the GEMM tiles, n_red_v of
  // them along the chunk rows; n_red = 0 when the reduction is a launch of its own
  int n_red, n_red_v;
  const float* part_db;
  int G_de, G_db, D;
  void* gE;
  int gE_dtype;
  float* gb;
  // the packing of the next chunk's W rows for the scores kernel (pack_rows_tile), as n_pack
  // workgroups after those, one 32-row x 8-slice tile per 256 threads at a time (n_pack_tiles in all)
  int n_pack, n_pack_tiles;
  const void* pk_src;  // W rows of the next chunk (fp32 when pk_f32, else the compute dtype)
  int pk_f32;
  int64_t pk_ld;
  int pk_rows, pk_S;
  void* pk_dst;        // their packed image
  void* pk_rowmajor;   // and the row-major copy in the compute dtype (fp32 W), or null
};

// Store 4 fp32 values as OutT (one 16- or 8-byte buffer store at byte offset
// voff of r; kOOB drops it).
template <class OutT>
__device__ __forceinline__ void store4_buf(__amdgpu_buffer_rsrc_t r, uint32_t voff, float4 v) {
  typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  if constexpr (sizeof(OutT) == 4) {
    const u32x4 u = {__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z), __float_as_uint(v.w)};
    __builtin_amdgcn_raw_buffer_store_b128(u, r, (int)voff, 0, 0);
  } else {
    OutT q[4] = {from_float<OutT>(v.x), from_float<OutT>(v.y), from_float<OutT>(v.z), from_float<OutT>(v.w)};
    u32x2 u;
    __builtin_memcpy(&u, q, 8);
    __builtin_amdgcn_raw_buffer_store_b64(u, r, (int)voff, 0, 0);
  }
}

// Store 4 fp32 values as OutT (one 16- or 8-byte store).
template <class OutT>
__device__ __forceinline__ void store4(OutT* dst, float4 v) {
  if constexpr (sizeof(OutT) == 4) {
    *reinterpret_cast<float4*>(dst) = v;
  } else {
    OutT q[4] = {from_float<OutT>(v.x), from_float<OutT>(v.y), from_float<OutT>(v.z), from_float<OutT>(v.w)};
    uint2 u;
    __builtin_memcpy(&u, q, 8);
    *reinterpret_cast<uint2*>(dst) = u;
  }
}

// Write a GEMM tile through LDS: out[(row_off + row) * ld + col] = fma(acc, scale,
// prev[...]) (prev = 0 when null) for rows < rows, cols < ld, with the tile at (tile_row0,
// tile_col0).  A lane's accumulators hold one column and 16 rows, so direct
// stores would be 2- or 4-byte pieces; instead each half of the tile (the
// rows of one wave row) is laid out row-major in LDS and written back by all
// threads as 16-byte chunks of whole rows.  prev (fp32, may alias out) is
// read per chunk just before the chunk is overwritten.  POS: the tile's rows
// are stage positions (tile_row0 multiple of 32), written to their tokens.
template <class G, int FM, int FN, bool POS = false, class OutT>
__device__ __forceinline__ void gemm_store(const f32x16_t (&acc)[FM][FN], float scale, OutT* out,
                                           const float* prev, int64_t row_off, int rows, int tile_row0,
                                           int tile_col0, int ld, char* smem) {
  constexpr int HALF = G::GM / G::WM, LSTR = G::GN + 8;  // rows per pass, floats per LDS row
  static_assert(HALF * LSTR * 4 <= G::EPI_BYTES, "epilogue fits in LDS");
  float* lds = reinterpret_cast<float*>(smem);
  // lane offsets from an opaque lane: computed here, not kept live through the reduction
  const int lane = lane_id() + opaque_zero(), w = wave_id(), wm = w / G::WN, wn = w % G::WN;
#pragma unroll
  for (int pass = 0; pass < G::WM; ++pass) {
    __syncthreads();  // every wave is done with the LDS (operand ring, or the previous pass)
    if (wm == pass) {
      // register r of a block holds row c_row(r, lane) = 4 hi + 8 (r / 4) + r % 4 (hi = lane / 32),
      // or for stage positions stage_tok of it = 8 hi + 16 ((r / 4) % 2) + 4 (r / 8) + r % 4:
      // one lane base, and a compile-time offset per register
      float* lb = lds + (POS ? 8 : 4) * (lane >> 5) * LSTR + wn * (G::GN / G::WN) + (lane & 31);
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < FN; ++fn)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int rc = POS ? 16 * ((r >> 2) & 1) + 4 * (r >> 3) + (r & 3) : 8 * (r >> 2) + (r & 3);
            lb[(fm * 32 + rc) * LSTR + fn * 32] = acc[fm][fn][r];
          }
    }
    __syncthreads();
    // Every chunk's previous value is requested before any is used, so the
    // read-modify-write costs one memory round trip per pass.  Loads and
    // stores are buffer operations with out-of-range chunks masked by offset,
    // not by branches: around divergent branches the compiler cannot count
    // the outstanding operations and waits for all of them before every add,
    // which would serialise the stores.
    constexpr int CPRW = G::GN / 4;               // 16-byte chunks per row
    constexpr int ITER = HALF * CPRW / G::NT;     // chunks per thread
    static_assert(HALF * CPRW % G::NT == 0, "whole chunks per thread");
    const int64_t first = (row_off + tile_row0 + pass * HALF) * ld + tile_col0;  // element of the pass's corner
    const __amdgpu_buffer_rsrc_t rp = buffer_rsrc(prev ? prev + first : nullptr);  // null prev: loads read zeros
    const __amdgpu_buffer_rsrc_t ro = buffer_rsrc(out + first);
    float4 pv[ITER];
    uint32_t el[ITER];  // element offset from the corner, or kOOB
#pragma unroll
    for (int i = 0; i < ITER; ++i) {
      const int c = i * G::NT + (int)threadIdx.x;
      const int rr = c / CPRW, c4 = c % CPRW;
      const int row = tile_row0 + pass * HALF + rr, col = tile_col0 + c4 * 4;
      // ld is a multiple of 8: a chunk is wholly in or out
      el[i] = row < rows && col < ld ? (uint32_t)(rr * ld + c4 * 4) : kOOB;
      const uint32_t vo = el[i] == kOOB ? kOOB : el[i] * 4;
      pv[i] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rp, (int)vo, 0, 0));
    }
#pragma unroll
    for (int i = 0; i < ITER; ++i) {
      const int c = i * G::NT + (int)threadIdx.x;
      float4 v = *reinterpret_cast<const float4*>(lds + (c / CPRW) * LSTR + (c % CPRW) * 4);
      // the scale is applied here, on the chunks being written, not to every accumulator at once
      v.x = fmaf(v.x, scale, pv[i].x);
      v.y = fmaf(v.y, scale, pv[i].y);
      v.z = fmaf(v.z, scale, pv[i].z);
      v.w = fmaf(v.w, scale, pv[i].w);
      store4_buf<OutT>(ro, el[i] == kOOB ? kOOB : el[i] * (uint32_t)sizeof(OutT), v);
    }
  }
}

// Tile loaders of the gradient GEMMs over the tiled stage (the LDS layouts of
// KTile / RTile, so the operand reads are the same).
// dW, A: rows = vocabulary rows from v0 (multiple of 32, rows_valid of them
// in the chunk), k = positions.
template <class T, int R, int BK, int NT>
struct StageKLoader {
  typedef KTile<T, R, BK, NT> Layout;
  static constexpr int BYTES = Layout::BYTES, NI = Layout::NI, NI_MIN = Layout::NI_MIN;
  static_assert(!Layout::PARTIAL && 32 % BK == 0, "whole loads, slices inside a block");
  const char* base;
  uint32_t off[NI];
  __device__ __forceinline__ void setup(const void* stage, int v0, int rows_valid, int n_tb32) {
    base = static_cast<const char*>(stage) + stage_off(v0, 0, n_tb32) * (int)sizeof(T);
#pragma unroll
    for (int i = 0; i < NI; ++i)
      off[i] = Layout::row_of(i) < rows_valid
                   ? (uint32_t)(stage_off(Layout::row_of(i), Layout::kc_of(i), n_tb32) * (int)sizeof(T))
                   : kOOB;
  }
  __device__ __forceinline__ void issue(uint32_t lds, int k0) const {
    const rsrc_t r = make_rsrc(base + ((int64_t)(k0 >> 5) * 1024 + (k0 & 31)) * (int)sizeof(T));
    dma_n<NI, NT * 16>(r, off, lds + wave_id() * 1024);
  }
};

// dh, A: rows = positions from q0 (multiple of 32), k = vocabulary rows,
// staged block-major (BRTile): a slice is R / 32 consecutive stage blocks, one
// contiguous run.  Every vocabulary row a slice reaches (below the chunk's
// rows rounded up to the scores tile) holds dS, zero past the chunk, so no
// bounds apply.
template <class T, int R, int BK, int NT>
struct StageBRLoader {
  typedef BRTile<T, R, BK, NT> Layout;
  static constexpr int BYTES = Layout::BYTES, NI = Layout::NI, NI_MIN = Layout::NI_MIN;
  static_assert(32 % BK == 0, "slices inside a block");
  const char* base;
  int n_tb32;
  uint32_t off[NI];
  __device__ __forceinline__ void setup(const void* stage, int q0, int ntb) {
    n_tb32 = ntb;
    base = static_cast<const char*>(stage) + stage_off(0, q0, ntb) * (int)sizeof(T);
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int lin = (i * NT + (int)threadIdx.x) * 16;  // byte in the tile image
      off[i] = (uint32_t)((lin / Layout::SUB) * 1024 * (int)sizeof(T) + lin % Layout::SUB);
    }
  }
  __device__ __forceinline__ void issue(uint32_t lds, int k0) const {
    const rsrc_t r = make_rsrc(base + stage_off(k0, 0, n_tb32) * (int)sizeof(T));
    dma_n<NI, NT * 16>(r, off, lds + wave_id() * 1024);
  }
};

// dW, B: h with the k-rows (tokens) of each 32-token block in position order.
template <class T, int R, int BK, int NT>
struct PosRLoader {
  typedef RTile<T, R, BK, NT> Layout;
  static constexpr int BYTES = Layout::BYTES, NI = Layout::NI, NI_MIN = Layout::NI_MIN;
  const char* base;
  int64_t ldb;
  int k_valid;
  uint32_t col[NI];  // column byte offset of this lane's chunk, or kOOB
  uint32_t off[NI];  // offset at a block start (k0 % 32 == 0), kOOB for absent columns
  __device__ __forceinline__ void setup(const T* b, int64_t ld, int cols_valid, int kv) {
    base = reinterpret_cast<const char*>(b);
    ldb = ld * (int64_t)sizeof(T);
    k_valid = kv;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int lin = (i * NT + (int)threadIdx.x) * 16;
      const int kr = lin / Layout::ROWB;
      const int r = (((lin % Layout::ROWB) / 16) ^ Layout::swz(kr)) * Layout::CE;
      col[i] = r < cols_valid ? (uint32_t)(r * (int)sizeof(T)) : kOOB;
      off[i] = r < cols_valid ? (uint32_t)(stage_tok(kr & 31) * ldb + r * (int)sizeof(T)) : kOOB;
    }
  }
  __device__ __forceinline__ void issue(uint32_t lds, int k0) const {
    const int kb = k0 & ~31;
    const rsrc_t rs = make_rsrc(base + (int64_t)kb * ldb);
    if (BK == 32 && kb + 32 <= k_valid) {
      dma_n<NI, NT * 16>(rs, off, lds + wave_id() * 1024);
    } else {
      uint32_t v[NI];
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int t = stage_tok((k0 & 31) + Layout::kr_of(i));
        v[i] = (col[i] == kOOB || kb + t >= k_valid) ? kOOB : (uint32_t)(t * ldb) + col[i];
      }
      dma_n<NI, NT * 16>(rs, v, lds + wave_id() * 1024);
    }
  }
};

// Single-tile pipelined reduction: acc += A[.., 0:k_total] B[.., 0:k_total]^T.
template <class T, int BK, int FM, int FN, class TA, class TB>
__device__ __forceinline__ void gemm_loop(f32x16_t (&acc)[FM][FN], const TA& ta, const TB& tb, char* smem,
                                          int k_total, int a_row0, int b_row0) {
  constexpr int SB = TA::BYTES + TB::BYTES;
  constexpr int L = TA::NI_MIN + TB::NI_MIN;  // conservative for partial tiles
  const int nk = (k_total + BK - 1) / BK;
  const uint32_t lds0 = lds_addr(smem);
  int is_k = 0, is_slot = 0;
  auto issue_next = [&]() {
    if (is_k >= nk) return;
    const uint32_t st = lds0 + is_slot * SB;
    ta.issue(st, is_k * BK);
    tb.issue(st + TA::BYTES, is_k * BK);
    ++is_k;
    is_slot = is_slot == kStages - 1 ? 0 : is_slot + 1;
  };
#pragma unroll
  for (int s = 0; s < kStages - 1; ++s) issue_next();
  if (nk == 0) return;
  Ring<kStages> ring{kStages - 1, nk};
  ring.publish_next<L>();
  tile_reduce<T, BK, L>(acc, ta, tb, smem, SB, ring, nk, a_row0, b_row0, issue_next);
}

// Tile of the gradient GEMMs: GM x GN per workgroup of WM x WN waves
// (two waves per SIMD for bf16 / f16, so one wave's LDS and barrier waits
// are covered by the other's matrix work).
template <class T>
struct GemmTile {
  static constexpr bool wide = sizeof(T) == 2;
  static constexpr int GM = wide ? 256 : 128;
  static constexpr int GN = GM;
  static constexpr int WM = 2;
  static constexpr int WN = wide ? 4 : 2;
  static constexpr int NT = 64 * WM * WN;
  // LDS: the operand ring, then (reused) the row-major epilogue staging of
  // half a tile in fp32 (rows padded by 8 floats: conflict-free writes)
  static constexpr int RING_BYTES = kStages * 2 * GM * SliceK<T>::value * (int)sizeof(T);
  static constexpr int EPI_BYTES = GM / WM * (GN + 8) * 4;
  static constexpr int LDS_BYTES = RING_BYTES > EPI_BYTES ? RING_BYTES : EPI_BYTES;
};

// One tile of one gradient product; DW selects the product (q: stage
// positions, tok(q) their tokens):
//   DW:  dW[v0+v][k]    = s sum_q stage[v][q] h[tok(q)][k]    (A: KTile layout, B: RTile layout)
//   !DW: dh[tok(q)][k] += s sum_v stage[v][q] W[v0+v][k]      (A: RTile layout, B: RTile layout)
template <class T, bool DW>
__device__ __forceinline__ void gemm_tile(const GemmParams& p, int t, char* smem) {
  typedef GemmTile<T> G;
  constexpr int kBK = SliceK<T>::value;
  constexpr int GM = G::GM, GN = G::GN, NT = G::NT;
  constexpr int FM = GM / (32 * G::WM), FN = GN / (32 * G::WN);
  const int w = wave_id();
  const int wm = w / G::WN, wn = w % G::WN;
  const int mt = t / p.n_n, nt = t % p.n_n;
  f32x16_t acc[FM][FN];
#pragma unroll
  for (int fm = 0; fm < FM; ++fm)
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) acc[fm][fn] = zero16();
  if constexpr (DW) {
    StageKLoader<T, GM, kBK, NT> ta;
    ta.setup(p.stage, mt * GM, p.cv - mt * GM, p.n_tb32);
    PosRLoader<T, GN, kBK, NT> tb;
    tb.setup(static_cast<const T*>(p.h) + nt * GN, p.ldh, p.K - nt * GN, p.N);
    // whole 32-position blocks of the active positions (padding positions
    // hold dS = 0 and zero rows of h)
    gemm_loop<T, kBK, FM, FN>(acc, ta, tb, smem, (min(p.N, p.n_act[0]) + 31) & ~31, wm * (GM / G::WM),
                              wn * (GN / G::WN));
  } else {
    StageBRLoader<T, GM, kBK, NT> ta;
    ta.setup(p.stage, mt * GM, p.n_tb32);
    RTile<T, GN, kBK, NT> tb;
    tb.setup(static_cast<const T*>(p.W) + (int64_t)(p.v0 - p.w_row0) * p.ldw + nt * GN, p.ldw, p.K - nt * GN, p.cv);
    gemm_loop<T, kBK, FM, FN>(acc, ta, tb, smem, p.cv, wm * (GM / G::WM), wn * (GN / G::WN));
  }
  const int rows = DW ? p.cv : p.N;
  const int row0 = mt * GM, col0 = nt * GN;
  // dispatch on the output dtype outside the unrolled store loops
  if constexpr (DW) {
    if (p.gW_dtype == kBF16)
      gemm_store<G>(acc, p.scale, static_cast<bf16_t*>(p.gW), nullptr, p.v0, rows, row0, col0, p.K, smem);
    else if (p.gW_dtype == kF16)
      gemm_store<G>(acc, p.scale, static_cast<f16_t*>(p.gW), nullptr, p.v0, rows, row0, col0, p.K, smem);
    else
      gemm_store<G>(acc, p.scale, static_cast<float*>(p.gW), nullptr, p.v0, rows, row0, col0, p.K, smem);
  } else {
    // dh over positions accumulates in fp32; bwd_expand_kernel writes gh
    const float* prev = p.dh_first ? nullptr : p.dh_acc;
    gemm_store<G, FM, FN, true>(acc, p.scale, p.dh_acc, prev, 0, rows, row0, col0, p.K, smem);
  }
}

// One tile of dE^T = gO^T P over one of de_split runs of the active positions (wide scores
// kernel): rows d (A: gO over positions read transposed, in stage position order), columns
// chunk-local vocabulary rows (B: the P stage), written as the run's fp32 partial [DP][C].  The
// runs are whole 32-position blocks; one past the active positions leaves its partial zero.  The
// split makes the dE^T work pieces of a tile, so a launch whose dW and dh tiles fill whole rounds
// of the CUs is not left a round of a few whole dE^T tiles; the partials are summed in run order
// by the reduction after the launch.
template <class T>
__device__ __forceinline__ void gemm_tile_de(const GemmParams& p, int t, char* smem) {
  typedef GemmTile<T> G;
  constexpr int kBK = SliceK<T>::value;
  constexpr int GM = G::GM, GN = G::GN, NT = G::NT;
  constexpr int FM = GM / (32 * G::WM), FN = GN / (32 * G::WN);
  const int w = wave_id();
  const int wm = w / G::WN, wn = w % G::WN;
  const int run = t % p.de_split;
  t /= p.de_split;
  const int mt = t / p.n_de_n, nt = t % p.n_de_n;
  const int kq = (min(p.N, p.n_act[0]) + 31) & ~31;        // active positions, whole blocks
  const int ks = ((kq + p.de_split - 1) / p.de_split + 31) & ~31;  // positions per run
  const int k0 = min(kq, run * ks), k1 = min(kq, k0 + ks);
  f32x16_t acc[FM][FN];
#pragma unroll
  for (int fm = 0; fm < FM; ++fm)
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) acc[fm][fn] = zero16();
  PosRLoader<T, GM, kBK, NT> ta;
  ta.setup(static_cast<const T*>(p.gOp) + (int64_t)k0 * p.DP + mt * GM, p.DP, p.DP - mt * GM, p.N - k0);
  StageKLoader<T, GN, kBK, NT> tb;
  tb.setup(p.pstage, nt * GN, p.cv - nt * GN, p.n_tb32);
  tb.base += (int64_t)(k0 >> 5) * 1024 * (int)sizeof(T);  // the run's first 32-position block
  gemm_loop<T, kBK, FM, FN>(acc, ta, tb, smem, k1 - k0, wm * (GM / G::WM), wn * (GN / G::WN));
  gemm_store<G>(acc, 1.f, p.part_dE + (int64_t)run * p.DP * p.C, nullptr, 0, p.DP, mt * GM, nt * GN, p.C, smem);
}

// Workgroup w of the W packing riding on a GEMM launch: tiles H i + part for i = w, w + n_pack, ...,
// each 256-thread part (H = NT / 256 of them) packing one tile through its own LDS block.
template <class T, int NT>
__device__ __forceinline__ void gemm_pack_w(const GemmParams& p, int w, char* smem) {
  constexpr int H = NT / 256;
  static_assert(NT % 256 == 0, "whole 256-thread parts");
  const int part = (int)threadIdx.x >> 8, t = (int)threadIdx.x & 255;
  uint4* tile = reinterpret_cast<uint4*>(smem) + part * (32 * 33);
  const int K = p.K;
  for (int i = w; H * i < p.n_pack_tiles; i += p.n_pack) {
    const int ti = H * i + part;
    const int grp_s = ti < p.n_pack_tiles ? ti : -1;
    if constexpr (sizeof(T) == 2) {
      if (p.pk_f32) {
        pack_rows_tile<float, T>(grp_s, t, tile, static_cast<const float*>(p.pk_src), p.pk_ld, p.pk_rows, K, p.pk_S,
                                 static_cast<T*>(p.pk_dst), static_cast<T*>(p.pk_rowmajor), nullptr, nullptr);
        __syncthreads();  // the next pair of tiles reuses the LDS blocks
        continue;
      }
    }
    pack_rows_tile<T, T>(grp_s, t, tile, static_cast<const T*>(p.pk_src), p.pk_ld, p.pk_rows, K, p.pk_S,
                         static_cast<T*>(p.pk_dst), nullptr, nullptr, nullptr);
    __syncthreads();  // the next pair of tiles reuses the LDS blocks
  }
}

// One launch covers the gradient products of a chunk: blocks [0, n_dw) are
// dW tiles, then n_de dE^T tiles (wide scores kernel only), then dh tiles.
// The dW and dE^T tiles (reductions over all active positions) are dealt first.
template <class T>
__global__ __launch_bounds__(GemmTile<T>::NT) void bwd_gemm_kernel(GemmParams p) {
  typedef GemmTile<T> G;
  constexpr int kBK = SliceK<T>::value;
  constexpr int SB = KTile<T, G::GM, kBK, G::NT>::BYTES + RTile<T, G::GN, kBK, G::NT>::BYTES;
  static_assert(KTile<T, G::GM, kBK, G::NT>::BYTES == RTile<T, G::GM, kBK, G::NT>::BYTES,
                "both A layouts stage the same bytes");
  static_assert(kStages * SB <= G::LDS_BYTES, "ring fits");
  __shared__ __attribute__((aligned(1024))) char smem[G::LDS_BYTES];
  int b = blockIdx.x;
  {
    // the dE / db reduction's workgroups, then the next chunk's W packing, follow every GEMM
    // tile: the dispatcher reaches them last, and they run on the CUs the last round of tiles
    // leaves idle
    const int r = b - (p.n_dw + p.n_de + p.n_dh);
    if (r >= 0 && r < p.n_red) {
      constexpr int RV = G::NT / 8;
      reduce_tile<G::NT>(reinterpret_cast<float(*)[kRedD + 1]>(smem), p.part_dE, p.part_db, p.G_de, p.G_db, p.C,
                         p.DP, p.v0, p.cv, p.D, p.gE, p.gE_dtype, p.gb, (r % p.n_red_v) * RV,
                         (r / p.n_red_v) * kRedD);
      return;
    }
    if (r >= p.n_red) {
      gemm_pack_w<T, G::NT>(p, r - p.n_red, smem);
      return;
    }
  }
  if (b < p.n_dw) {
    int r, c;
    grouped_tile(b, p.n_dw / p.n_n, p.n_n, &r, &c);
    gemm_tile<T, true>(p, r * p.n_n + c, smem);
    return;
  }
  b -= p.n_dw;
  if (b < p.n_de) {
    gemm_tile_de<T>(p, b, smem);
    return;
  }
  b -= p.n_de;
  {
    // dh tiles of the active positions' row blocks only (the grid covers all
    // of N); the active tiles are spread over every XCD
    const int n_dh = min(p.n_dh, (p.n_act[0] + G::GM - 1) / G::GM * p.n_n);
    if (b < n_dh) {
      int r, c;
      grouped_tile(b, n_dh / p.n_n, p.n_n, &r, &c);
      gemm_tile<T, false>(p, r * p.n_n + c, smem);
    }
  }
}

__global__ __launch_bounds__(256) void bwd_reduce_kernel(const float* __restrict__ part_dE,
                                                         const float* __restrict__ part_db, int G_de, int G, int C,
                                                         int DP, int v0, int cv, int D, void* gE, int gE_dtype,
                                                         float* gb) {
  __shared__ float tile[kRedV][kRedD + 1];  // padded: the transposed accesses stay conflict-free
  reduce_tile<256>(tile, part_dE, part_db, G_de, G, C, DP, v0, cv, D, gE, gE_dtype, gb, blockIdx.x * kRedV,
                   blockIdx.y * kRedD);
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

// The narrow-embedding scores kernel (side tiles carried by the ring) serves
// bf16 / f16 with DP <= 64; the general one serves the rest.
template <class T, int DP>
struct ScoresRing {
  static constexpr bool value = sizeof(T) == 2 && DP <= 64;
};

template <class T, int DP, bool F8 = false>
hipError_t launch_scores(const BwdPlan& plan, const ScoresParams& sp, hipStream_t stream) {
  if constexpr (ScoresRing<T, DP>::value) {
    typedef ScoresRingTile<T, DP> C;
    if (plan.BM != C::BM || plan.BV != C::BV || plan.kind != kScoresRing) return hipErrorInvalidValue;
    timing_begin(kKindBwdScores, stream);
    bwd_scores_ring_kernel<T, DP, F8><<<sp.n_vtc * sp.G, C::NT, 0, stream>>>(sp);
    timing_end(kKindBwdScores, stream);
  } else {
    typedef ScoresTile<T, DP> C;
    if (plan.BM != C::BM || plan.BV != C::BV || plan.kind != kScoresGeneral) return hipErrorInvalidValue;
    timing_begin(kKindBwdScores, stream);
    bwd_scores_kernel<T, DP, F8><<<sp.n_vtc * sp.G, C::NT, 0, stream>>>(sp);
    timing_end(kKindBwdScores, stream);
  }
  return hipGetLastError();
}

template <class T>
hipError_t dispatch_scores(const BwdPlan& plan, const ScoresParams& sp, hipStream_t stream) {
  if (plan.kind == kScoresWide) {
    typedef ScoresWideTile<T> C;
    if (sp.multp || plan.BM != C::BM || plan.BV != C::BV || plan.DP % SliceK<T>::value != 0)
      return hipErrorInvalidValue;
    timing_begin(kKindBwdScores, stream);
    bwd_scores_wide_kernel<T><<<sp.n_vtc * sp.G, C::NT, 0, stream>>>(sp);
    timing_end(kKindBwdScores, stream);
    return hipGetLastError();
  }
  if constexpr (std::is_same<T, bf16_t>::value) {
    if (sp.multp) {  // e4m3 scores (bf16 compute dtype only)
      switch (plan.DP) {
        case 32: return launch_scores<T, 32, true>(plan, sp, stream);
        case 64: return launch_scores<T, 64, true>(plan, sp, stream);
        case 128: return launch_scores<T, 128, true>(plan, sp, stream);
        default: return hipErrorInvalidValue;
      }
    }
  }
  if (sp.multp) return hipErrorInvalidValue;
  switch (plan.DP) {  // 2-byte dtypes: the ring kernel (DP <= 64); fp32: the general one (DP <= 128)
    case 32: return launch_scores<T, 32>(plan, sp, stream);
    case 64: return launch_scores<T, 64>(plan, sp, stream);
    case 128:
      if constexpr (sizeof(T) == 4) return launch_scores<T, 128>(plan, sp, stream);
      return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
}

template <class T>
hipError_t dispatch_gemm(const BwdPlan& plan, const GemmParams& gp, hipStream_t stream) {
  const int blocks = gp.n_dw + gp.n_de + gp.n_dh + gp.n_red + gp.n_pack;
  if (blocks == 0) return hipSuccess;
  if (plan.GM != GemmTile<T>::GM || plan.GN != GemmTile<T>::GN) return hipErrorInvalidValue;
  timing_begin(kKindBwdGemm, stream);
  bwd_gemm_kernel<T><<<blocks, GemmTile<T>::NT, 0, stream>>>(gp);
  timing_end(kKindBwdGemm, stream);
  return hipGetLastError();
}

template <class T>
hipError_t bwd_run(const BwdPlan& plan, const BwdParams& p, hipStream_t stream) {
  hipError_t e;
  char* ws = p.ws;
  T* stage = reinterpret_cast<T*>(ws + plan.off_stage);
  T* pstage = plan.kind == kScoresWide ? reinterpret_cast<T*>(ws + plan.off_pstage) : nullptr;
  float* part_dE = reinterpret_cast<float*>(ws + plan.off_pe);
  float* part_db = reinterpret_cast<float*>(ws + plan.off_pb);
  float* dh_acc = plan.dh_acc ? reinterpret_cast<float*>(ws + plan.off_dh) : nullptr;
  T* gOp = reinterpret_cast<T*>(ws + plan.off_gO);
  T* gOt = reinterpret_cast<T*>(ws + plan.off_gOt);
  float* lsed = reinterpret_cast<float*>(ws + plan.off_lsed);
  T* Ep = reinterpret_cast<T*>(ws + plan.off_Ep);
  float* biasp = reinterpret_cast<float*>(ws + plan.off_bias);
  T* hp = reinterpret_cast<T*>(ws + plan.off_hp);
  T* Wp = reinterpret_cast<T*>(ws + plan.off_Wp);
  int* flag = reinterpret_cast<int*>(ws + plan.off_flag);
  int* idx = reinterpret_cast<int*>(ws + plan.off_idx);
  int* inv = reinterpret_cast<int*>(ws + plan.off_inv);
  int* n_act = reinterpret_cast<int*>(ws + plan.off_nact);
  float* delta = reinterpret_cast<float*>(ws + plan.off_delta);
  T* hc = reinterpret_cast<T*>(ws + plan.off_hc);
  // W in the compute dtype, row-major, as the dh product reads it: the caller's, or for an fp32 W
  // a copy made while packing, chunk c's rows in buffer c % 2 (the launch that reads chunk c
  // writes chunk c + 1's rows)
  T* Wc = (sizeof(T) == 2 && p.w_f32) ? reinterpret_cast<T*>(ws + plan.off_Wc) : nullptr;
  auto wc_buf = [&](int c) { return Wc + (int64_t)(c & 1) * plan.C * p.K; };
  // e4m3 scores: e4m3 h over positions (bytes, read as K8 / 2 pairs) and the per-row multipliers
  const bool f8 = p.hq != nullptr;
  T* hqc = reinterpret_cast<T*>(ws + plan.off_hqc);
  float* multp = f8 ? reinterpret_cast<float*>(ws + plan.off_mult) : nullptr;
  const bool need_stage = p.gh || p.gW;
  const bool gemm_de = pstage && p.gE;  // dE^T = gO^T P as tiles of the gradient GEMM launch
  // every chunk has a gradient GEMM launch: the W packing of the scores kernel rides on them
  const bool fold_pack = !f8 && (need_stage || gemm_de);

  {
    // delta, the active tokens, and the token-side operands over positions
    timing_begin(kKindBwdDelta, stream);
    bwd_delta_kernel<T><<<(p.N + 255) / 256, 256, 0, stream>>>(p.O, p.gO, p.glse, p.N, p.D, delta, flag);
    bwd_compact_kernel<<<1, 1024, 0, stream>>>(flag, p.N, idx, inv, n_act);
    const int64_t n = (int64_t)plan.N_pad * plan.DP;
    bwd_pack_kernel<T><<<(int)((n + 255) / 256), 256, 0, stream>>>(p.gO, p.lse, delta, idx, n_act, p.D,
                                                                   (int)plan.N_pad, plan.DP, plan.BM, gOp, gOt,
                                                                   lsed);
    timing_end(kKindBwdDelta, stream);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    const int64_t nv = (int64_t)plan.V_pad * plan.DP;
    timing_begin(kKindPack, stream);
    pack_vocab_kernel<T><<<(int)((nv + 255) / 256), 256, 0, stream>>>(
        static_cast<const T*>(p.E), p.lde, p.bias, p.V, p.D, plan.V_pad, plan.DP, Ep, biasp, p.h_scale, p.w_scale,
        p.scale, multp);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if (p.K > 0) {
      const int64_t nh = plan.N_pad * (p.K / (16 / (int)sizeof(T)));
      const unsigned gb = (unsigned)((nh + 255) / 256);
      if (sizeof(T) == 2 && p.h_f32)
        bwd_gather_rows_kernel<float, T><<<gb, 256, 0, stream>>>(static_cast<const float*>(p.h), p.ldh, idx,
                                                                  n_act, (int)plan.N_pad, p.K, hc);
      else
        bwd_gather_rows_kernel<T, T><<<gb, 256, 0, stream>>>(static_cast<const T*>(p.h), p.ldh, idx, n_act,
                                                              (int)plan.N_pad, p.K, hc);
      if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    if (f8) {
      // the scores kernel reads the e4m3 operands; the gradient GEMMs keep h over positions and W
      const int k2 = p.K8 / 2;
      const int64_t nq = plan.N_pad * (k2 / (16 / (int)sizeof(T)));
      bwd_gather_rows_kernel<T, T><<<(unsigned)((nq + 255) / 256), 256, 0, stream>>>(
          static_cast<const T*>(p.hq), p.ldhq / 2, idx, n_act, (int)plan.N_pad, k2, hqc);
      if ((e = hipGetLastError()) != hipSuccess) return e;
      if ((e = launch_pack_rows<T>(hqc, k2, (int)plan.N_pad, k2, plan.hS8, plan.N_pad, hp, stream)) != hipSuccess)
        return e;
      if ((e = pack_src<T>(p.Wq, false, p.ldwq / 2, p.V, k2, plan.hS8, plan.V_pad, Wp, stream, nullptr)) !=
          hipSuccess)
        return e;
    } else {
      if ((e = launch_pack_rows<T>(hc, p.K, (int)plan.N_pad, p.K, plan.hS, plan.N_pad, hp, stream)) != hipSuccess)
        return e;
      // Wp holds one chunk's packed rows: the first chunk's are packed here; chunk c + 1's by
      // chunk c's gradient GEMM launch (gemm_pack_w) after chunk c's scores kernel has read its
      // own, or, without gradient GEMM launches, before chunk c + 1's scores kernel.  fp32 W: the
      // packing also writes the row-major copy the dh product reads.
      const int64_t rows0 = p.V < plan.C ? p.V : plan.C;
      const int64_t pad0 = (rows0 + plan.BV - 1) / plan.BV * plan.BV;
      if ((e = pack_src<T>(p.W, p.w_f32, p.ldw, (int)rows0, p.K, plan.hS, pad0, Wp, stream,
                           fold_pack ? Wc : nullptr)) != hipSuccess)
        return e;
    }
    timing_end(kKindPack, stream);
  }

  for (int c = 0; c < plan.n_chunks; ++c) {
    const int v0 = (int)(c * plan.C);
    const int cv = (int)((p.V - v0) < plan.C ? (p.V - v0) : plan.C);
    // A partial last chunk has fewer vocabulary tiles: more token groups fill the chip with it
    // (G from the same rule as the plan's).  Its partials use its own width as their row stride,
    // so G_c x width stays within the buffers' G x C.
    const int n_vtc = (cv + plan.BV - 1) / plan.BV;
    const int Cc = n_vtc * plan.BV;
    int Gc = plan.wgs == 256 ? plan.wgs / n_vtc : (plan.wgs + n_vtc - 1) / n_vtc;
    if (Gc > plan.n_tb) Gc = plan.n_tb;
    if ((int64_t)Gc * Cc > (int64_t)plan.G * plan.C) Gc = (int)((int64_t)plan.G * plan.C / Cc);
    if (Gc < plan.G) Gc = plan.G;  // a full chunk: the plan's G
    const int n_gpart_c = plan.n_gpart / plan.G * Gc;
    if (!f8 && !fold_pack && c > 0) {
      timing_begin(kKindPack, stream);
      e = pack_src<T>(static_cast<const char*>(p.W) + (int64_t)v0 * p.ldw * (p.w_f32 ? 4 : (int64_t)sizeof(T)),
                      p.w_f32, p.ldw, cv, p.K, plan.hS, Cc, Wp, stream, nullptr);
      timing_end(kKindPack, stream);
      if (e != hipSuccess) return e;
    }
    ScoresParams sp;
    sp.hp = hp;
    // e4m3: Wp holds every row's packed image; the kernels address the chunk's rows from row v0
    sp.Wp = f8 ? Wp + (int64_t)v0 * plan.hS8 * SliceK<T>::value : Wp;
    sp.hS = f8 ? plan.hS8 : plan.hS;
    sp.Ep = Ep;
    sp.biasp = biasp;
    sp.multp = multp;
    sp.scale = p.scale;
    sp.N = p.N;
    sp.K = f8 ? p.K8 / 2 : p.K;
    sp.gOp = gOp;
    sp.gOt = gOt;
    sp.lsed = lsed;
    sp.N_pad = (int)plan.N_pad;
    sp.v0 = v0;
    sp.cv = cv;
    sp.C = Cc;
    sp.n_tb = plan.n_tb;
    sp.G = Gc;
    sp.n_vtc = n_vtc;
    sp.stage = stage;
    sp.pstage = pstage;
    sp.n_tb32 = (int)(plan.N_pad / 32);
    sp.part_dE = part_dE;
    sp.part_db = part_db;
    sp.need_stage = need_stage;
    sp.need_dE = p.gE != nullptr;
    sp.need_db = p.gb != nullptr;
    sp.n_act = n_act;
    sp.DP = plan.DP;
    if ((e = dispatch_scores<T>(plan, sp, stream)) != hipSuccess) return e;

    bool fold_red = false;
    if (need_stage || gemm_de) {
      GemmParams gp;
      gp.stage = stage;
      gp.n_tb32 = (int)(plan.N_pad / 32);
      gp.N_pad = plan.N_pad;
      gp.h = hc;
      gp.ldh = p.K;
      gp.W = Wc ? static_cast<const void*>(wc_buf(c)) : p.W;
      gp.ldw = Wc ? p.K : p.ldw;
      gp.w_row0 = Wc ? v0 : 0;
      gp.N = p.N;
      gp.K = p.K;
      gp.v0 = v0;
      gp.cv = cv;
      gp.n_n = (p.K + plan.GN - 1) / plan.GN;
      gp.n_dw = p.gW ? ((cv + plan.GM - 1) / plan.GM) * gp.n_n : 0;
      gp.n_dh = p.gh ? ((p.N + plan.GM - 1) / plan.GM) * gp.n_n : 0;
      gp.n_de_n = (cv + plan.GN - 1) / plan.GN;
      gp.de_split = de_split(plan.N_pad);
      gp.n_de = gemm_de ? ((plan.DP + plan.GM - 1) / plan.GM) * gp.n_de_n * gp.de_split : 0;
      gp.pstage = pstage;
      gp.gOp = gOp;
      gp.DP = plan.DP;
      gp.part_dE = part_dE;
      gp.C = Cc;
      gp.gW = p.gW;
      gp.gW_dtype = p.gW_dtype;
      gp.dh_acc = dh_acc;
      gp.dh_first = c == 0;
      gp.scale = p.scale;
      gp.n_act = n_act;
      // the reduction of the scores kernel's partials rides on this launch (the wide kernel's dE^T
      // is formed in it, so that reduction follows as a launch of its own)
      fold_red = (p.gE || p.gb) && !gemm_de;
      gp.n_red_v = (cv + GemmTile<T>::NT / 8 - 1) / (GemmTile<T>::NT / 8);
      gp.n_red = fold_red ? gp.n_red_v * (p.gE && p.D > 0 ? (p.D + kRedD - 1) / kRedD : 1) : 0;
      gp.part_db = part_db;
      gp.G_de = n_gpart_c;
      gp.G_db = n_gpart_c;
      gp.D = p.D;
      gp.gE = p.gE;
      gp.gE_dtype = p.gE_dtype;
      gp.gb = p.gb;
      // the next chunk's W rows into the scores kernel's packed image (and the row-major copy of
      // an fp32 W), as in the packing before the loop
      gp.n_pack = gp.n_pack_tiles = 0;
      if (fold_pack && c + 1 < plan.n_chunks) {
        const int64_t v1 = v0 + plan.C;
        const int cv1 = (int)((p.V - v1) < plan.C ? (p.V - v1) : plan.C);
        const int pad1 = (cv1 + plan.BV - 1) / plan.BV * plan.BV;
        constexpr int H = GemmTile<T>::NT / 256;
        const bool f32src = sizeof(T) == 2 && p.w_f32;
        gp.pk_f32 = f32src;
        gp.pk_src = static_cast<const char*>(p.W) + v1 * p.ldw * (f32src ? 4 : (int64_t)sizeof(T));
        gp.pk_ld = p.ldw;
        gp.pk_rows = cv1;
        gp.pk_S = plan.hS;
        gp.pk_dst = Wp;
        gp.pk_rowmajor = Wc ? wc_buf(c + 1) : nullptr;
        gp.n_pack_tiles = (pad1 / 32) * ((plan.hS + 7) / 8);
        const int iters = (gp.n_pack_tiles + H - 1) / H;
        gp.n_pack = iters < 1024 ? iters : 1024;
      }
      if ((e = dispatch_gemm<T>(plan, gp, stream)) != hipSuccess) return e;
    }
    if ((p.gE || p.gb) && !fold_red) {
      timing_begin(kKindBwdReduce, stream);
      const dim3 grid((unsigned)((cv + kRedV - 1) / kRedV),
                      p.gE && p.D > 0 ? (unsigned)((p.D + kRedD - 1) / kRedD) : 1u);
      bwd_reduce_kernel<<<grid, 256, 0, stream>>>(
          part_dE, part_db, plan.kind == kScoresWide ? de_split(plan.N_pad) : n_gpart_c, n_gpart_c, Cc, plan.DP, v0, cv,
          p.D, p.gE, p.gE_dtype, p.gb);
      timing_end(kKindBwdReduce, stream);
      if ((e = hipGetLastError()) != hipSuccess) return e;
    }
  }
  if (p.gh) {
    const int64_t ng = (int64_t)p.N * (p.K / 4);
    if (ng > 0) {
      timing_begin(kKindBwdExpand, stream);
      bwd_expand_kernel<<<(int)((ng + 255) / 256), 256, 0, stream>>>(dh_acc, inv, p.N, p.K, p.gh, p.gh_dtype);
      timing_end(kKindBwdExpand, stream);
      if ((e = hipGetLastError()) != hipSuccess) return e;
    }
  }
  return hipSuccess;
}

// Tile of the scores kernel that serves (T, DP), and how many workgroups a
// chunk should have: one per CU for the ring and wide kernels (one fits a
// CU), two per CU for the general one.
template <class T, int DP>
void general_tile(int* BM, int* BV, int* WT, int* wgs) {
  *BM = ScoresTile<T, DP>::BM;
  *BV = ScoresTile<T, DP>::BV;
  *WT = ScoresTile<T, DP>::WT;
  *wgs = 512;
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

size_t dtype_bytes(int dtype) { return dtype == kF32 ? 4 : 2; }

}  // namespace

hipError_t compact_tokens(const int* flag, int N, int* idx, int* inv, int* n_act, hipStream_t stream) {
  bwd_compact_kernel<<<1, 1024, 0, stream>>>(flag, N, idx, inv, n_act);
  return hipGetLastError();
}

bool bwd_plan(int dtype, int64_t N, int64_t K, int64_t V, int64_t D, int64_t chunk, bool need_gh, BwdPlan* plan,
              bool w_f32, int64_t K8) {
  const bool f8 = K8 > 0;
  if (f8 && (dtype != kBF16 || D > 128 || K8 % 16 != 0)) return false;
  const bool two = dtype == kBF16 || dtype == kF16;
  if (!two && dtype != kF32) return false;
  // Padded embedding width and scores kernel:
  //   2-byte dtypes: the ring kernel up to 64; above, the wide kernel (any multiple of 32),
  //     but the e4m3 scores, which keep the general kernel at 128;
  //   fp32: the general kernel up to 128; above, the wide kernel (any multiple of 16).
  int DP, kind;
  if (D <= 64) {
    DP = D <= 32 ? 32 : 64;
    kind = two ? kScoresRing : kScoresGeneral;
  } else if (f8 || (!two && D <= 128)) {
    DP = 128;
    kind = kScoresGeneral;
  } else {
    const int64_t sw = two ? 32 : 16;
    DP = (int)((D + sw - 1) / sw * sw);
    kind = kScoresWide;
  }
  int BM, BV, WT, wgs;
  if (kind == kScoresRing) {
    BM = ScoresRingTile<bf16_t, 64>::BM;
    BV = ScoresRingTile<bf16_t, 64>::BV;
    WT = ScoresRingTile<bf16_t, 64>::WT;
    wgs = 256;
  } else if (kind == kScoresWide) {
    BM = two ? ScoresWideTile<bf16_t>::BM : ScoresWideTile<float>::BM;
    BV = ScoresWideTile<bf16_t>::BV;
    WT = ScoresWideTile<bf16_t>::WT;
    wgs = 256;  // one workgroup per CU (its ring takes 132 KB of LDS, fp32 100 KB)
  } else if (two) {
    general_tile<bf16_t, 128>(&BM, &BV, &WT, &wgs);
  } else if (DP == 32) {
    general_tile<float, 32>(&BM, &BV, &WT, &wgs);
  } else if (DP == 64) {
    general_tile<float, 64>(&BM, &BV, &WT, &wgs);
  } else {
    general_tile<float, 128>(&BM, &BV, &WT, &wgs);
  }
  const int GM = two ? GemmTile<bf16_t>::GM : GemmTile<float>::GM;
  const int GN = two ? GemmTile<bf16_t>::GN : GemmTile<float>::GN;
  plan->DP = DP;
  plan->BM = BM;
  plan->BV = BV;
  plan->GM = GM;
  plan->GN = GN;
  plan->n_tb = (int)((N + BM - 1) / BM);
  plan->N_pad = ((N + 255) / 256) * 256;
  if (plan->N_pad == 0) plan->N_pad = 256;
  int64_t c = chunk < V ? chunk : V;
  // at most 2^22 rows per chunk: tile-relative offsets into [DP or rows][C] buffers stay 32-bit
  if (c > ((int64_t)1 << 22)) c = (int64_t)1 << 22;
  if (c < 1) c = 1;
  c = ((c + BV - 1) / BV) * BV;
  plan->C = c;
  plan->n_chunks = (int)((V + c - 1) / c);
  const int n_vtc = (int)(c / BV);
  int G = wgs == 256 ? wgs / n_vtc : (wgs + n_vtc - 1) / n_vtc;
  if (G > plan->n_tb) G = plan->n_tb;
  if (G < 1) G = 1;
  plan->G = G;
  plan->wgs = wgs;
  plan->n_gpart = G * WT;  // db (and, but for the wide kernel, dE) partials: one per token group and token-wave row
  plan->kind = kind;
  plan->dh_acc = need_gh;
  plan->V_pad = ((V + BV - 1) / BV) * BV;
  const size_t tb = dtype_bytes(dtype);
  size_t off = 0;
  plan->off_stage = off;
  off += align256((size_t)c * (size_t)plan->N_pad * tb);
  plan->off_pe = off;
  off += align256((size_t)(kind == kScoresWide ? de_split(plan->N_pad) : plan->n_gpart) * DP * c * 4);
  plan->off_pstage = off;
  if (kind == kScoresWide) off += align256((size_t)c * (size_t)plan->N_pad * tb);
  plan->off_pb = off;
  off += align256((size_t)plan->n_gpart * c * 4);
  plan->off_dh = off;
  if (plan->dh_acc) off += align256((size_t)N * K * 4);
  plan->off_gO = off;
  off += align256((size_t)plan->N_pad * DP * tb);
  plan->off_gOt = off;
  off += align256((size_t)plan->N_pad * DP * tb);
  plan->off_lsed = off;
  off += align256((size_t)plan->N_pad * 2 * 4);
  plan->off_Ep = off;
  off += align256((size_t)plan->V_pad * DP * tb);
  plan->off_bias = off;
  off += align256((size_t)plan->V_pad * 4);
  const int bk = dtype == kF32 ? SliceK<float>::value : SliceK<bf16_t>::value;
  plan->hS = packed_slices(K, bk);
  plan->hS8 = K8 > 0 ? packed_slices(K8 / 2, bk) : 0;
  const int hs_max = plan->hS > plan->hS8 ? plan->hS : plan->hS8;
  plan->off_hp = off;
  off += align256((size_t)plan->N_pad * hs_max * bk * tb);
  // packed W: one chunk's rows (the e4m3 scores: every row's, packed once)
  plan->off_Wp = off;
  off += align256((size_t)(K8 > 0 ? plan->V_pad : c) * hs_max * bk * tb);
  plan->off_flag = off;
  off += align256((size_t)plan->N_pad * 4);
  plan->off_idx = off;
  off += align256((size_t)plan->N_pad * 4);
  plan->off_inv = off;
  off += align256((size_t)plan->N_pad * 4);
  plan->off_nact = off;
  off += 256;
  plan->off_delta = off;
  off += align256((size_t)plan->N_pad * 4);
  plan->off_hc = off;
  off += align256((size_t)plan->N_pad * K * tb);
  // fp32 W: its compute-dtype rows of two chunks (one when there is one chunk)
  plan->off_Wc = off;
  if (w_f32 && tb == 2) off += align256((size_t)(plan->n_chunks > 1 ? 2 : 1) * c * K * tb);
  plan->off_hqc = off;  // e4m3 h over positions, K8 bytes per row
  if (K8 > 0) off += align256((size_t)plan->N_pad * K8);
  plan->off_mult = off;
  if (K8 > 0) off += align256((size_t)plan->V_pad * 4);
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
