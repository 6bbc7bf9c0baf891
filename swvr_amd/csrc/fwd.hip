// Fused forward: O = softmax(s * h W^T + b) E and LSE, without writing scores.
//
// Algorithm: the online softmax of swvr/chunked.py:82-105 (docs/DESIGN.md:12-24),
// reorganised for the GPU:
//   * a workgroup owns BM tokens and one of n_split contiguous vocabulary
//     ranges; it walks that range BV rows at a time;
//   * per vocabulary tile it forms S^T = W_tile h_tile^T (BV x BM) with MFMA
//     over the whole hidden size K, streaming K slices of the packed W and h
//     through an NS-slot LDS ring (3 slots beside the pinned E^T tile for
//     2-byte dtypes with D <= 64, 4 for fp32; for 2-byte D of 128 and 256
//     E^T travels through the ring instead, 3 stages of two slices each,
//     fwd_stream_kernel);
//   * the waves form a WV (vocabulary) x WT (tokens) grid: at D <= 64, 8 waves
//     of 128 vocabulary rows x 64 tokens (2 x 4) over a 256 x 256 tile.  In
//     the S^T layout each lane holds one token column, so the softmax max/sum
//     over the vocabulary is a register reduction plus one lane swap;
//   * every wave keeps its own running (m, l, acc) over its half of each tile
//     (an independent partial softmax), and P, rounded to the compute dtype as
//     the reference rounds it (swvr/chunked.py:103, triton_kernels.py:69),
//     feeds acc^T += E^T P^T straight from the score registers;
//   * partials (m, l, acc) of all waves and splits are merged by
//     fwd_combine_kernel in a fixed order (deterministic).
#include <cmath>
#include <type_traits>

#include "common.hpp"
#include "launch.hpp"

namespace swvr {

namespace {

// Tile shape per (dtype, padded D): BV vocabulary rows x BM tokens per
// workgroup of WV x WT waves (two waves per SIMD for bf16 / f16); the
// per-wave score block and acc^T block share the register file, NS K-slices
// of W and h plus the E^T tile and the bias share LDS (160 KB).  For the
// narrow embeddings (DP <= 64) each wave owns 128 vocabulary rows x 64
// tokens: 0.75 operand reads per MFMA.
template <class T, int DP>
struct FwdTile {
  static constexpr bool wide = sizeof(T) == 2;
  static constexpr bool narrow = wide && DP <= 64;
  // D = 128 and 256 (2-byte dtypes): E^T streamed through the ring in D-slices (fwd_stream_kernel)
  static constexpr bool stream_e = wide && (DP == 256 || DP == 128);
  // 2-byte dtypes: 128 x 64 waves (D <= 64), 128 x 32 (D = 128 and 256, E^T streamed): the widest
  // whose score and acc^T accumulators fit beside the operands at D = 256; at D = 128 they run
  // 2% faster than 64 x 64 waves with E^T pinned
  static constexpr int BV = wide ? 256 : 128;
  static constexpr int BM = narrow ? 256 : wide ? 128 : 64;
  static constexpr int WV = 2;
  static constexpr int WT = narrow ? 4 : wide ? 4 : 2;
  static constexpr int NT = 64 * WV * WT;
  static constexpr int NS = narrow ? 3 : kStages;  // LDS ring depth of fwd_tile_kernel (160 KB with E^T)
};

// The e4m3 forward (h and W in OCP e4m3, E and P in bf16): one k64 MFMA per
// 64-byte slice takes 32 operand bytes per lane, twice the bf16 k16 step's, so
// the 128 x 64 wave of the bf16 tile would not fit its accumulators and
// operands in 256 registers.  D <= 64: waves of 64 x 64 (one operand read per
// MFMA), a 4-deep ring of 24 KB slices and the software-pipelined reduction
// (two operand sets).  D = 128 (wider E^T tile and accumulators): 128 x 32
// waves, 3 slices, one operand set.
static_assert(kFP8 == kFwdFP8, "one dtype code for the e4m3 forward");

template <int DP>
struct FwdTileF8 {
  static constexpr bool pipe = DP <= 64;
  static constexpr int BV = 256, BM = 128, WV = pipe ? 4 : 2, WT = pipe ? 2 : 4;
  static constexpr int NT = 64 * WV * WT;
  static constexpr int NS = pipe ? 4 : 3;
};

template <class T, int DP, bool F8>
using FwdCfg = typename std::conditional<F8, FwdTileF8<DP>, FwdTile<T, DP>>::type;

// Vocabulary operands of the forward, packed once per call: E^T per
// vocabulary tile as [n_vt][DP][BV] (compute dtype; column p of tile vt is
// row vt * BV + pe_row(p) of E; zero past D and V) and the bias as fp32
// [V_pad] (-inf past V: padding rows drop out of the softmax).
// With w_scale set (the e4m3 forward) the bias goes out as (bias, multiplier)
// pairs, multiplier = logit_scale * h_scale * w_scale[v] (0 past V): the
// factor that turns the e4m3 dot product into a score.
template <class T>
__global__ __launch_bounds__(256) void pack_et_kernel(const T* __restrict__ E, int64_t lde,
                                                      const float* __restrict__ bias, int V, int D, int V_pad,
                                                      int DP, int BV, T* __restrict__ Et, float* __restrict__ biasp,
                                                      const float* __restrict__ h_scale,
                                                      const float* __restrict__ w_scale, float logit_scale) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e < (int64_t)V_pad * DP) {
    const int64_t tile = e / ((int64_t)DP * BV);
    const int rem = (int)(e - tile * DP * BV);
    const int d = rem / BV, p = rem % BV;
    const int64_t v = tile * BV + pe_row(p);
    Et[e] = (v < V && d < D) ? E[v * lde + d] : (T)0.f;
  }
  if (e < V_pad) {
    const float b = e < V ? (bias ? bias[e] : 0.f) : kNegInf;
    if (w_scale) {
      biasp[2 * e] = b;
      biasp[2 * e + 1] = e < V ? logit_scale * h_scale[0] * w_scale[e] : 0.f;
    } else {
      biasp[e] = b;
    }
  }
}


template <class T, int DP, bool F8 = false>
__global__ __launch_bounds__((FwdCfg<T, DP, F8>::NT)) void fwd_tile_kernel(FwdParams p) {
  typedef FwdCfg<T, DP, F8> C;
  typedef typename Vec8<T>::type V8;
  constexpr int kBK = SliceK<T>::value;
  constexpr int BV = C::BV, BM = C::BM, NT = C::NT;
  constexpr int WVR = BV / C::WV, WTR = BM / C::WT;  // rows per wave
  typedef PackedKLoader<T, BV, kBK, NT> TA;  // W rows of the vocabulary tile (packed)
  typedef PackedKLoader<T, BM, kBK, NT> TB;  // h rows of the token block (packed)
  typedef KTile<T, DP, BV, NT> TE;   // E^T tile [DP][BV] in pe_row order, swizzled like an operand tile
  constexpr int SB = TA::BYTES + TB::BYTES;
  constexpr int L = TA::NI_MIN + TB::NI_MIN;  // conservative for partial tiles
  constexpr int FV = WVR / 32, FT = WTR / 32;  // 32x32 blocks per wave
  constexpr int DB = DP / 32;
  constexpr int EBYTES = TE::BYTES;
  constexpr int BBYTES = BV * 4 * (F8 ? 2 : 1);  // bias, or (bias, multiplier) pairs

  constexpr int NS = C::NS;
  __shared__ __attribute__((aligned(1024))) char smem[NS * SB + EBYTES + BBYTES];
  char* const sE = smem + NS * SB;
  const float* const sBias = reinterpret_cast<const float*>(sE + EBYTES);

  const int lane = lane_id(), w = (int)(threadIdx.x >> 6);
  const int wv = w / C::WT, wt = w % C::WT;
  int n_tb = p.n_tb, n_split = p.n_split, ntok = p.N;  // ntok: token rows of a partial
  if (p.n_act) {
    n_tb = p.n_act[3];
    n_split = p.n_act[4];
    if ((int)blockIdx.x >= n_tb * n_split) return;
    ntok = n_tb * BM;
  }
  int split, tb;
  grouped_tile(blockIdx.x, n_split, n_tb, &split, &tb);
  const int n0 = tb * BM;
  const int vt_begin = (int)((int64_t)split * p.n_vt / n_split);
  const int vt_end = (int)((int64_t)(split + 1) * p.n_vt / n_split);
  const T* Ep = static_cast<const T*>(p.Ep);

  float m[FT], l[FT];
  f32x16_t oacc[DB][FT];
#pragma unroll
  for (int ft = 0; ft < FT; ++ft) {
    m[ft] = kNegInf;
    l[ft] = 0.f;
#pragma unroll
    for (int db = 0; db < DB; ++db) oacc[db][ft] = zero16();
  }

  const int nk = max(1, (p.K + kBK - 1) / kBK);  // K = 0: one all-zero slice (bias-only scores)
  const int n_tiles = vt_end - vt_begin;
  const uint32_t lds0 = lds_addr(smem);
  const uint32_t ldsE = lds0 + NS * SB, ldsB = ldsE + EBYTES;
  TA ta;
  ta.setup(p.Wp, vt_begin * BV, p.hS);
  TB tbh;
  tbh.setup(p.hp, n0, p.hS);
  // issue cursor: the next stage to load (NS - 1 ahead of the compute)
  int is_tile = 0, is_kt = 0, is_slot = 0;
  auto issue_next = [&]() {
    if (is_tile >= n_tiles) return;
    if (is_kt == 0) {
      const int v0 = (vt_begin + is_tile) * BV;
      ta.rebase(v0);
    }
    const uint32_t st = lds0 + is_slot * SB;
    ta.issue(st, is_kt * kBK);
    tbh.issue(st + TA::BYTES, is_kt * kBK);
    if (++is_kt == nk) {
      is_kt = 0;
      ++is_tile;
    }
    is_slot = is_slot == NS - 1 ? 0 : is_slot + 1;
  };
#pragma unroll
  for (int s = 0; s < NS - 1; ++s) issue_next();

  f32x16_t sacc[FV][FT];
  Ring<NS> ring{NS - 1, n_tiles * nk};  // the first publish_next() moves to stage 0, slot 0
  for (int tile = 0; tile < n_tiles; ++tile) {
    const int v0 = (vt_begin + tile) * BV;
    // first stage of the tile; every wave has also finished the previous
    // tile's epilogue, so the E and bias tiles can be replaced
    ring.template publish_next<L>();
    {
      TE te;
      te.setup(Ep + (int64_t)v0 * DP, BV, DP, BV);
      te.issue(ldsE, 0);
      if ((int)threadIdx.x * 16 < BBYTES)
        dma_batch1(make_rsrc(p.biasp + (int64_t)v0 * (F8 ? 2 : 1)), (uint32_t)threadIdx.x * 16, ldsB + w * 1024);
    }
#pragma unroll
    for (int fv = 0; fv < FV; ++fv)
#pragma unroll
      for (int ft = 0; ft < FT; ++ft) sacc[fv][ft] = zero16();
    if constexpr (F8)
      tile_reduce_f8<L, FwdTileF8<DP>::pipe>(sacc, ta, tbh, smem, SB, ring, nk, wv * WVR, wt * WTR, issue_next);
    else
      tile_reduce<T, kBK, L>(sacc, ta, tbh, smem, SB, ring, nk, wv * WVR, wt * WTR, issue_next);
    if (nk < NS) {
      // short reduction: the E / bias loads may still be in flight
      wait_vmcnt<0>();
      stage_barrier();
    }

    // ---- scores -> running softmax of this wave's slice of the tile
    float mx[FT];
#pragma unroll
    for (int ft = 0; ft < FT; ++ft) mx[ft] = kNegInf;
#pragma unroll
    for (int fv = 0; fv < FV; ++fv)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        // registers 4g..4g+3 hold rows 8g + 4(lane/32) + 0..3 of the block
        const int row = wv * WVR + fv * 32 + 8 * g + (lane >> 5) * 4;
        float bb[4], mm[4];
        if constexpr (F8) {
          const float4 x0 = *reinterpret_cast<const float4*>(sBias + 2 * row);
          const float4 x1 = *reinterpret_cast<const float4*>(sBias + 2 * row + 4);
          bb[0] = x0.x; mm[0] = x0.y; bb[1] = x0.z; mm[1] = x0.w;
          bb[2] = x1.x; mm[2] = x1.y; bb[3] = x1.z; mm[3] = x1.w;
        } else {
          const float4 b4 = *reinterpret_cast<const float4*>(sBias + row);
          bb[0] = b4.x; bb[1] = b4.y; bb[2] = b4.z; bb[3] = b4.w;
          mm[0] = mm[1] = mm[2] = mm[3] = p.scale;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int ft = 0; ft < FT; ++ft) {
            const float x = fmaf(sacc[fv][ft][4 * g + i], mm[i], bb[i]);  // rounded as the backward rounds it
            sacc[fv][ft][4 * g + i] = x;
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
    // they hold vocabulary rows 16c + 8(t/4) + 4(lane/32) + t%4, t = 0..7,
    // which the packed E^T tile stores contiguously (pe_row): one read per
    // operand.
    const char* sEe = sE + opaque_zero();  // read base, recomputed per tile
#pragma unroll
    for (int fv = 0; fv < FV; ++fv)
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        V8 av[DB];
        const int p0 = wv * WVR + fv * 32 + 8 * (2 * c + (lane >> 5));
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const int d = db * 32 + (lane & 31);
          if constexpr (sizeof(T) == 2) {
            av[db] = *reinterpret_cast<const V8*>(sEe + TE::elem(d, p0));
          } else {
            const float4 lo = *reinterpret_cast<const float4*>(sEe + TE::elem(d, p0));
            const float4 hi = *reinterpret_cast<const float4*>(sEe + TE::elem(d, p0 + 4));
            av[db][0] = lo.x; av[db][1] = lo.y; av[db][2] = lo.z; av[db][3] = lo.w;
            av[db][4] = hi.x; av[db][5] = hi.y; av[db][6] = hi.z; av[db][7] = hi.w;
          }
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

  // ---- partial (m, l, acc) of this wave's vocabulary slice of this split
  // (lane offsets from an opaque lane: computed here, not kept live through the loop)
  const int part = split * C::WV + wv;
  const int ln = lane + opaque_zero();
#pragma unroll
  for (int ft = 0; ft < FT; ++ft) {
    const int n = n0 + wt * WTR + ft * 32 + (ln & 31);
    if (n < ntok) {
      if (ln < 32) {
        p.part_m[(int64_t)part * ntok + n] = m[ft];
        p.part_l[(int64_t)part * ntok + n] = l[ft];
      }
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int d = db * 32 + c_row(r, ln);
          p.part_acc[((int64_t)part * DP + d) * ntok + n] = oacc[db][ft][r];
        }
    }
  }
}

// Forward for D = 128 and 256 (2-byte dtypes): E^T is not pinned in LDS.  Per
// vocabulary tile the ring carries the K-slices of W and h (-> S^T), then the
// DP / 32 D-slices of the tile's packed E^T (32 x BV each, 16 KB), so the LDS
// holds only the ring: 256 vocabulary rows x 128 tokens per workgroup of 8
// waves (2 vocabulary halves x 4 token quarters, 128 x 32 each); at D = 256
// that is twice the tile a pinned E^T tile would leave room for (85 flop per
// byte of operand traffic instead of 64).  Each of the ring's 3 stages holds two slices (48 KB: two
// K-slices, or two D-slices), so the wait + barrier that publishes a stage
// comes once per 128 MFMAs of the workgroup, as in the 256 x 256 tile of the
// narrow forward.  The bias of a tile is loaded with its first K-slices into a
// double-buffered strip.
template <class T, int DP>
__global__ __launch_bounds__((FwdTile<T, DP>::NT)) void fwd_stream_kernel(FwdParams p) {
  typedef FwdTile<T, DP> C;
  typedef typename Vec8<T>::type V8;
  constexpr int kBK = SliceK<T>::value;
  constexpr int BV = C::BV, BM = C::BM, NT = C::NT;
  constexpr int NS = 3, P = 2;  // ring stages, slices per stage
  constexpr int WVR = BV / C::WV, WTR = BM / C::WT;  // rows per wave
  typedef PackedKLoader<T, BV, kBK, NT> TA;  // W rows of the vocabulary tile (packed)
  typedef PackedKLoader<T, BM, kBK, NT> TB;  // h rows of the token block (packed)
  constexpr int DS = 32;                     // E^T rows (embedding columns) per D-slice
  typedef KTile<T, DS, BV, NT> TE;           // one D-slice of the packed E^T tile, pe_row order
  constexpr int SB1 = TA::BYTES + TB::BYTES; // one slice
  constexpr int SB = P * SB1;                // one stage
  constexpr int L1 = TA::NI + TB::NI;        // loads per thread per slice (E^T slices padded to it)
  constexpr int L = P * L1;                  // per stage
  static_assert(sizeof(T) == 2 && DP % (DS * P) == 0 && TE::BYTES <= SB1 && TE::NI <= L1, "E^T slices fit");
  static_assert(L1 * NT * 16 == SB1, "a slice's loads fill its bytes");
  static_assert(!TA::PARTIAL && !TB::PARTIAL && !TE::PARTIAL, "whole loads");
  constexpr int FV = WVR / 32, FT = WTR / 32;  // 32x32 blocks per wave
  constexpr int DB = DP / 32, ND = DP / DS, NE = ND / P;

  __shared__ __attribute__((aligned(1024))) char smem[NS * SB + 2 * BV * 4];
  const float* const sBias = reinterpret_cast<const float*>(smem + NS * SB);  // [2][BV]

  const int lane = lane_id(), w = wave_id();
  const int wv = w / C::WT, wt = w % C::WT;
  int n_tb = p.n_tb, n_split = p.n_split, ntok = p.N;  // ntok: token rows of a partial
  if (p.n_act) {
    n_tb = p.n_act[3];
    n_split = p.n_act[4];
    if ((int)blockIdx.x >= n_tb * n_split) return;
    ntok = n_tb * BM;
  }
  int split, tb;
  // per XCD, 2 vocabulary splits x 16 token blocks at D = 256, 1 x 32 at D = 128 (each 1-2% faster
  // than the other there)
  grouped_tile<DP == 128 ? 1 : 2>(blockIdx.x, n_split, n_tb, &split, &tb);
  const int n0 = tb * BM;
  const int vt_begin = (int)((int64_t)split * p.n_vt / n_split);
  const int vt_end = (int)((int64_t)(split + 1) * p.n_vt / n_split);
  const T* Ep = static_cast<const T*>(p.Ep);

  float m[FT], l[FT];
  f32x16_t oacc[DB][FT];
#pragma unroll
  for (int ft = 0; ft < FT; ++ft) {
    m[ft] = kNegInf;
    l[ft] = 0.f;
#pragma unroll
    for (int db = 0; db < DB; ++db) oacc[db][ft] = zero16();
  }

  const int nk = max(1, (p.K + kBK - 1) / kBK);  // K = 0: one all-zero slice (bias-only scores)
  const int nkst = (nk + P - 1) / P;             // K-stages per tile; an odd nk leaves a zero slice
  const int n_tiles = vt_end - vt_begin;
  const int per_tile = nkst + NE;
  const int total = n_tiles * per_tile;
  const uint32_t lds0 = lds_addr(smem);
  const uint32_t ldsB = lds0 + NS * SB;
  TA ta;
  ta.setup(p.Wp, vt_begin * BV, p.hS);
  TB tbh;
  tbh.setup(p.hp, n0, p.hS);
  TE te;
  te.setup(Ep, BV, DS, BV);
  const rsrc_t r_none = make_rsrc(nullptr);
  auto zero_fill = [&](int from, uint32_t st) {  // zero-filling loads from..L1-1 of a slice
#pragma unroll
    for (int i = 0; i < L1; ++i)
      if (i >= from) dma_batch1(r_none, kOOB, st + i * NT * 16 + w * 1024);
  };
  // issue cursor over the walk: stage `issued` is (tile is_tile, sub-stage
  // is_sub) into slot is_slot; sub-stages 0..nkst-1 hold K-slices 2 sub and
  // 2 sub + 1, nkst.. D-slices 2 e and 2 e + 1 of the tile's E^T
  int issued = 0, is_tile = 0, is_sub = 0, is_slot = 0;
  auto issue_next = [&]() {
    if (issued >= total) return;
    const uint32_t st = lds0 + is_slot * SB;
    const int v0 = (vt_begin + is_tile) * BV;
    if (is_sub < nkst) {
      if (is_sub == 0) {
        ta.rebase(v0);
        // the tile's bias into strip (tile & 1), ahead of its slices (wave 0)
        if ((int)threadIdx.x * 16 < BV * 4)
          dma_batch1(make_rsrc(p.biasp + v0), (uint32_t)threadIdx.x * 16, ldsB + (is_tile & 1) * (BV * 4) + w * 1024);
      }
#pragma unroll
      for (int s = 0; s < P; ++s) {
        const int k = P * is_sub + s;
        const uint32_t ss = st + s * SB1;
        if (k < nk) {
          ta.issue(ss, k * kBK);
          tbh.issue(ss + TA::BYTES, k * kBK);
        } else {
          zero_fill(0, ss);
        }
      }
    } else {
      // rows d0 .. d0 + 31 of the tile's E^T [DP][BV]: one contiguous run per D-slice
#pragma unroll
      for (int s = 0; s < P; ++s) {
        const int ds = P * (is_sub - nkst) + s;
        const uint32_t ss = st + s * SB1;
        te.base = reinterpret_cast<const char*>(Ep + ((int64_t)v0 * DP + (int64_t)ds * DS * BV));
        te.issue(ss, 0);
        zero_fill(TE::NI, ss);
      }
    }
    ++issued;
    if (++is_sub == per_tile) {
      is_sub = 0;
      ++is_tile;
    }
    is_slot = is_slot == NS - 1 ? 0 : is_slot + 1;
  };
#pragma unroll
  for (int s = 0; s < NS - 1; ++s) issue_next();

  f32x16_t sacc[FV][FT];
  Ring<NS> ring{NS - 1, total};  // the first publish_next() moves to stage 0, slot 0
  for (int tile = 0; tile < n_tiles; ++tile) {
    // first K-stage of the tile; every wave has also finished the previous
    // tile's E^T slices, and its bias strip is free again
    ring.template publish_next<L>();
#pragma unroll
    for (int fv = 0; fv < FV; ++fv)
#pragma unroll
      for (int ft = 0; ft < FT; ++ft) sacc[fv][ft] = zero16();
    tile_reduce_multi<T, kBK, P, L>(sacc, ta, tbh, smem, SB, SB1, ring, nkst, wv * WVR, wt * WTR, issue_next);

    // ---- scores -> running softmax of this wave's slice of the tile
    const float* sB = sBias + (tile & 1) * BV + opaque_zero();
    float mx[FT];
#pragma unroll
    for (int ft = 0; ft < FT; ++ft) mx[ft] = kNegInf;
#pragma unroll
    for (int fv = 0; fv < FV; ++fv)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        // registers 4g..4g+3 hold rows 8g + 4(lane/32) + 0..3 of the block
        const int row = wv * WVR + fv * 32 + 8 * g + (lane >> 5) * 4;
        const float4 b4 = *reinterpret_cast<const float4*>(sB + row);
        const float bb[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int ft = 0; ft < FT; ++ft) {
            const float x = fmaf(sacc[fv][ft][4 * g + i], p.scale, bb[i]);  // rounded as the backward rounds it
            sacc[fv][ft][4 * g + i] = x;
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

    // ---- acc^T[d][token] += E^T[d][v] P^T[v][token], two D-slices per stage.
    // Score registers 8c..8c+7 of a block are the B operand of one k16 step;
    // they hold vocabulary rows 16c + 8(t/4) + 4(lane/32) + t%4, which the
    // packed E^T stores contiguously (pe_row): one read per operand.
#pragma unroll
    for (int e = 0; e < NE; ++e) {
      ring.template publish_next<L>();
      issue_next();
      const int d = lane & 31;
#pragma unroll
      for (int s = 0; s < P; ++s) {
        const char* sEe = smem + ring.slot * SB + s * SB1 + opaque_zero();
#pragma unroll
        for (int fv = 0; fv < FV; ++fv)
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            const int p0 = wv * WVR + fv * 32 + 8 * (2 * c + (lane >> 5));
            const V8 av = *reinterpret_cast<const V8*>(sEe + TE::elem(d, p0));
#pragma unroll
            for (int ft = 0; ft < FT; ++ft) {
              V8 bv;
#pragma unroll
              for (int tt = 0; tt < 8; ++tt) bv[tt] = from_float<T>(sacc[fv][ft][8 * c + tt]);
              mfma_k16(oacc[P * e + s][ft], av, bv);
            }
          }
      }
    }
  }

  // ---- partial (m, l, acc) of this wave's vocabulary slice of this split
  const int part = split * C::WV + wv;
  const int ln = lane + opaque_zero();
#pragma unroll
  for (int ft = 0; ft < FT; ++ft) {
    const int n = n0 + wt * WTR + ft * 32 + (ln & 31);
    if (n < ntok) {
      if (ln < 32) {
        p.part_m[(int64_t)part * ntok + n] = m[ft];
        p.part_l[(int64_t)part * ntok + n] = l[ft];
      }
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int d = db * 32 + c_row(r, ln);
          p.part_acc[((int64_t)part * DP + d) * ntok + n] = oacc[db][ft][r];
        }
    }
  }
}

// Merge partial softmaxes in a fixed order (O rows ldo apart): O = sum_p acc_p e^(m_p - M) /
// sum_p l_p e^(m_p - M), LSE = M + log(...).  A row with every score -inf ends
// with M = -inf, L = 0: O = NaN and LSE = -inf, as swvr/chunked.py:105 gives.
// Partial p of (row n, column d) of acc sits at p * sp + d * sd + n * sn, so
// one kernel merges the forward's own partials ([n_part][DP][N], token
// fastest) and vocabulary shards' ([S][N][D]).  With m_out set, it writes the
// merged partial (M, L and the unnormalised acc, [N][D]) instead of O / LSE.
// One thread per (d, n) with n fastest; the d = 0 thread of a row also writes
// its LSE (or M, L).
// Merge of one (row, column) over n_part partials: m / l of partial q at
// pm[q * sml] / pl[q * sml], its acc at pa[q * sp] (read when has_d).  The
// loads go out in batches of 8 ahead of the arithmetic, which runs in partial
// order, so the merge waits for memory once per batch, not once per partial.
__device__ __forceinline__ void merge_partials(const float* __restrict__ pm, const float* __restrict__ pl,
                                               const float* __restrict__ pa, int n_part, int64_t sml, int64_t sp,
                                               bool has_d, float* M_, float* L_, float* a_) {
  constexpr int B = 8;
  float M = kNegInf;
  for (int q0 = 0; q0 < n_part; q0 += B) {
    float x[B];
#pragma unroll
    for (int u = 0; u < B; ++u) x[u] = q0 + u < n_part ? pm[(q0 + u) * sml] : kNegInf;
#pragma unroll
    for (int u = 0; u < B; ++u) M = fmaxf(M, x[u]);
  }
  const float shift = M == kNegInf ? 0.f : M;
  float L = 0.f, a = 0.f;
  for (int q0 = 0; q0 < n_part; q0 += B) {
    float xm[B], xl[B], xa[B];
#pragma unroll
    for (int u = 0; u < B; ++u) {
      const bool in = q0 + u < n_part;
      xm[u] = in ? pm[(q0 + u) * sml] : 0.f;
      xl[u] = in ? pl[(q0 + u) * sml] : 0.f;
      xa[u] = in && has_d ? pa[(q0 + u) * sp] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < B; ++u)
      if (q0 + u < n_part) {
        const float wq = expf(xm[u] - shift);
        L += xl[u] * wq;
        if (has_d) a += xa[u] * wq;
      }
  }
  *M_ = M;
  *L_ = L;
  *a_ = a;
}

__global__ __launch_bounds__(256) void fwd_combine_kernel(const float* __restrict__ part_m,
                                                          const float* __restrict__ part_l,
                                                          const float* __restrict__ part_acc, int n_part, int N,
                                                          int D, int64_t sp, int64_t sd, int64_t sn,
                                                          float* __restrict__ O, int64_t ldo, float* __restrict__ lse,
                                                          float* __restrict__ m_out, float* __restrict__ l_out) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int Dw = D > 0 ? D : 1;
  if (e >= (int64_t)N * Dw) return;
  const int d = (int)(e / N), n = (int)(e % N);
  float M, L, a;
  merge_partials(part_m + n, part_l + n, part_acc + d * sd + n * sn, n_part, N, sp, d < D, &M, &L, &a);
  if (m_out) {
    if (d < D) O[(int64_t)n * ldo + d] = a;
    if (d == 0) {
      m_out[n] = M;
      l_out[n] = L;
    }
  } else {
    if (d < D) O[(int64_t)n * ldo + d] = a / L;
    if (d == 0) lse[n] = M + logf(L);
  }
}

// fwd_combine_kernel of the active-token forward: token n merges the partials
// of its position inv[n] (WV x n_split partials of n_tb x BM rows each, n_tb and
// n_split at n_act[3], n_act[4]); a token outside the active set gets an O row
// of 0 and LSE 0.
__global__ __launch_bounds__(256) void fwd_combine_active_kernel(
    const float* __restrict__ part_m, const float* __restrict__ part_l, const float* __restrict__ part_acc,
    const int* __restrict__ inv, const int* __restrict__ n_act, int BM, int WV, int N, int D, int DP,
    float* __restrict__ O, int64_t ldo, float* __restrict__ lse) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int Dw = D > 0 ? D : 1;
  if (e >= (int64_t)N * Dw) return;
  const int d = (int)(e / N), n = (int)(e % N);
  const int q = inv[n];
  if (q < 0) {
    if (d < D) O[(int64_t)n * ldo + d] = 0.f;
    if (d == 0) lse[n] = 0.f;
    return;
  }
  const int tb = n_act[3], sp = n_act[4];
  const int64_t rows = (int64_t)tb * BM;
  float M, L, a;
  merge_partials(part_m + q, part_l + q, part_acc + d * rows + q, WV * sp, rows, (int64_t)DP * rows, d < D, &M, &L,
                 &a);
  if (d < D) O[(int64_t)n * ldo + d] = a / L;
  if (d == 0) lse[n] = M + logf(L);
}

// The active-token forward's token blocks and vocabulary splits (active_grid)
// from the count, into n_act[3], n_act[4]: once per call, for every kernel.
__global__ __launch_bounds__(64) void fwd_active_grid_kernel(int* __restrict__ n_act, int BM, int n_tb_max,
                                                             int n_split0, int n_vt) {
  if (threadIdx.x == 0) {
    int tb, sp;
    active_grid(n_act[0], BM, n_tb_max, n_split0, n_vt, &tb, &sp);
    n_act[3] = tb;
    n_act[4] = sp;
  }
}

// Flags of the active-token forward's parameter checks, bad[0..1]:
// bad[0] = 1 when the logit scale is not finite, E holds an infinity or a NaN
// or the bias a NaN or +inf (W is checked as it is packed); bad[1] starts at 1
// when there is a bias (or no vocabulary) and drops to 0 once a bias entry
// above -inf is seen (every entry -inf makes every score -inf).
__global__ __launch_bounds__(64) void fwd_flags_init_kernel(int* __restrict__ bad, int scale_bad, int bias_all_neg) {
  if (threadIdx.x == 0) {
    bad[0] = scale_bad;
    bad[1] = bias_all_neg;
  }
}

// Grid-stride scan of E's V x D elements and the bias for fwd_flags_init_kernel's
// words.  Every store writes the same value, so the words end the same
// whatever the order of the stores.
template <class T>
__global__ __launch_bounds__(256) void fwd_param_scan_kernel(const T* __restrict__ E, int64_t lde, int V, int D,
                                                             const float* __restrict__ bias, int* __restrict__ bad) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t t0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  bool nf = false, live = false;
  if (D > 0)
    for (int64_t e = t0; e < (int64_t)V * D; e += stride) {
      const int64_t v = e / D;
      nf |= !__builtin_isfinite((float)E[v * lde + (e - v * D)]);
    }
  if (bias)
    for (int64_t v = t0; v < V; v += stride) {
      const float b = bias[v];
      nf |= b != b || b == kPosInf;
      live |= b > kNegInf;
    }
  if (__syncthreads_or(nf) && threadIdx.x == 0) bad[0] = 1;
  if (__syncthreads_or(live) && threadIdx.x == 0) bad[1] = 0;
}

// flag[n] = 1 for a token of the active-token forward: a non-zero (or NaN)
// weight, an h row holding an infinity or a NaN (in the compute dtype), or a
// flagged parameter (bad[0] or bad[1]: then every token).  One wave per token;
// only a zero-weight token's row is read, in 16-byte chunks.
template <class Src, class T>
__global__ __launch_bounds__(256) void fwd_active_flag_kernel(const float* __restrict__ weight,
                                                              const Src* __restrict__ h, int64_t ldh, int N, int K,
                                                              const int* __restrict__ bad, int* __restrict__ flag) {
  const int n = blockIdx.x * 4 + (int)(threadIdx.x >> 6);
  if (n >= N) return;
  const int lane = lane_id();
  bool act = weight[n] != 0.f || bad[0] != 0 || bad[1] != 0;  // NaN != 0
  if (!act) {  // uniform over the wave
    constexpr int CE = 16 / (int)sizeof(T);
    bool nf = false;
    for (int c = lane; c < K / CE; c += 64)
      nf |= chunk_nonfinite<T>(load_chunk<Src, T>(h + (int64_t)n * ldh + (int64_t)c * CE));
    act = __ballot(nf) != 0;
  }
  if (lane == 0) flag[n] = act ? 1 : 0;
}

template <class T, int DP, bool F8 = false>
hipError_t launch_tile(const FwdPlan& plan, const FwdParams& p, hipStream_t stream) {
  typedef FwdCfg<T, DP, F8> C;
  if (plan.BV != C::BV || plan.BM != C::BM) return hipErrorInvalidValue;
  // the active-token forward may use up to twice the all-token grid (active_grid); the rest exit at once
  const int blocks = plan.n_tb * plan.n_split * (p.n_act ? 2 : 1);
  timing_begin(kKindFwdTile, stream);
  if constexpr (!F8 && FwdTile<T, DP>::stream_e)
    fwd_stream_kernel<T, DP><<<blocks, C::NT, 0, stream>>>(p);
  else
    fwd_tile_kernel<T, DP, F8><<<blocks, C::NT, 0, stream>>>(p);
  timing_end(kKindFwdTile, stream);
  return hipGetLastError();
}

template <class T>
hipError_t dispatch_dp(const FwdPlan& plan, const FwdParams& p, hipStream_t stream) {
  switch (plan.DP) {
    case 32: return launch_tile<T, 32>(plan, p, stream);
    case 64: return launch_tile<T, 64>(plan, p, stream);
    case 128: return launch_tile<T, 128>(plan, p, stream);
    case 256:
      if constexpr (sizeof(T) == 2) return launch_tile<T, 256>(plan, p, stream);
      return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
}

hipError_t dispatch_dp_f8(const FwdPlan& plan, const FwdParams& p, hipStream_t stream) {
  switch (plan.DP) {
    case 32: return launch_tile<bf16_t, 32, true>(plan, p, stream);
    case 64: return launch_tile<bf16_t, 64, true>(plan, p, stream);
    case 128: return launch_tile<bf16_t, 128, true>(plan, p, stream);
    default: return hipErrorInvalidValue;
  }
}

template <class T, int DP>
void tile_get(int* BV, int* BM, int* WV) {
  *BV = FwdTile<T, DP>::BV;
  *BM = FwdTile<T, DP>::BM;
  *WV = FwdTile<T, DP>::WV;
}

template <class T>
void tile_of(int DP, int* BV, int* BM, int* WV) {
  switch (DP) {
    case 32: tile_get<T, 32>(BV, BM, WV); break;
    case 64: tile_get<T, 64>(BV, BM, WV); break;
    case 128: tile_get<T, 128>(BV, BM, WV); break;
    default: tile_get<T, 256>(BV, BM, WV); break;
  }
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// E^T tiles and the bias of one D-slice (p.E, p.D: the slice's columns).
template <class T>
hipError_t pack_et(const FwdParams& p, const FwdPlan& plan, hipStream_t stream) {
  const int64_t n = (int64_t)plan.V_pad * plan.DP;
  timing_begin(kKindPack, stream);
  pack_et_kernel<T><<<(int)((n + 255) / 256), 256, 0, stream>>>(
      static_cast<const T*>(p.E), p.lde, p.bias, p.V, p.D, plan.V_pad, plan.DP, plan.BV,
      const_cast<T*>(static_cast<const T*>(p.Ep)), const_cast<float*>(p.biasp), p.h_scale, p.w_scale, p.scale);
  timing_end(kKindPack, stream);
  return hipGetLastError();
}

// h and W in their tiles' LDS image, once per call.
template <class T>
hipError_t pack(const FwdParams& p, const FwdPlan& plan, hipStream_t stream) {
  timing_begin(kKindPack, stream);
  hipError_t e = hipSuccess;
  T* const hp = const_cast<T*>(static_cast<const T*>(p.hp));
  T* const Wp = const_cast<T*>(static_cast<const T*>(p.Wp));
  if (e == hipSuccess)
    e = pack_src<T>(p.h, p.h_f32, p.ldh, p.N, p.K, plan.hS, plan.N_pad, hp, stream);
  if (e == hipSuccess)
    e = pack_src<T>(p.W, p.w_f32, p.ldw, p.V, p.K, plan.hS, plan.V_pad, Wp, stream);
  timing_end(kKindPack, stream);
  return e;
}

}  // namespace

bool fwd_plan(int dtype, int64_t N, int64_t K, int64_t V, int64_t D, FwdPlan* plan, bool active) {
  (void)K;
  if (active && dtype == kFP8) return false;
  plan->active = active;
  // Widest embedding slice of one pass: 256 (2-byte dtypes), 128 (fp32, e4m3).  A wider D runs
  // in slices of that width, each pass recomputing the same scores for its columns of E.
  const int DS = dtype == kBF16 || dtype == kF16 ? 256 : 128;
  if (dtype == kFP8 && D > DS) return false;
  const int64_t Dw = D < DS ? D : DS;
  const int DP = Dw <= 32 ? 32 : Dw <= 64 ? 64 : Dw <= 128 ? 128 : 256;
  plan->DS = DS;
  plan->n_dslices = D > DS ? (int)((D + DS - 1) / DS) : 1;
  int BV, BM, WV;
  size_t tbytes;
  if (dtype == kF32) {
    if (DP > 128) return false;
    tile_of<float>(DP, &BV, &BM, &WV);
    tbytes = 4;
  } else if (dtype == kBF16 || dtype == kF16) {
    tile_of<bf16_t>(DP, &BV, &BM, &WV);
    tbytes = 2;
  } else if (dtype == kFP8) {
    // K counts byte pairs: the e4m3 rows are packed as bf16 rows of K / 2 elements
    if (DP > 128) return false;
    static_assert(FwdTileF8<128>::BV == FwdTileF8<64>::BV && FwdTileF8<128>::BM == FwdTileF8<64>::BM, "one tile");
    BV = FwdTileF8<64>::BV;
    BM = FwdTileF8<64>::BM;
    WV = DP <= 64 ? FwdTileF8<64>::WV : FwdTileF8<128>::WV;
    tbytes = 2;
  } else {
    return false;
  }
  plan->BV = BV;
  plan->BM = BM;
  plan->DP = DP;
  plan->n_tb = (int)((N + BM - 1) / BM);
  plan->n_vt = (int)((V + BV - 1) / BV);
  plan->V_pad = plan->n_vt * BV;
  // Enough workgroups (one per CU) to fill 256 CUs several times over, at
  // least two vocabulary tiles per split.
  int n_split = 1;
  if (plan->n_tb > 0) {
    const int target = 1024;
    n_split = (target + plan->n_tb - 1) / plan->n_tb;
    const int max_split = plan->n_vt / 2 > 1 ? plan->n_vt / 2 : 1;
    if (n_split > max_split) n_split = max_split;
    if (n_split < 1) n_split = 1;
  }
  plan->n_split = n_split;
  plan->n_part = WV * n_split;
  plan->WV = WV;
  // token rows of a partial: N; the active-token forward's partials hold up to
  // 2 x n_tb x n_split workgroups' n_tb x BM positions each (active_grid)
  const int64_t NR = active ? 2 * (int64_t)plan->n_tb * BM : N;
  size_t off = 0;
  plan->off_m = off;
  off += align256((size_t)plan->n_part * NR * 4);
  plan->off_l = off;
  off += align256((size_t)plan->n_part * NR * 4);
  plan->off_acc = off;
  off += align256((size_t)plan->n_part * NR * 4 * DP);
  plan->off_Ep = off;
  off += align256((size_t)plan->V_pad * DP * tbytes);
  plan->off_bias = off;
  off += align256((size_t)plan->V_pad * 4 * (dtype == kFP8 ? 2 : 1));
  plan->N_pad = ((N + 255) / 256) * 256;
  plan->hS = packed_slices(K, tbytes == 4 ? SliceK<float>::value : SliceK<bf16_t>::value);
  plan->off_hp = off;
  off += align256((size_t)plan->N_pad * plan->hS * (tbytes == 4 ? SliceK<float>::value : SliceK<bf16_t>::value) * tbytes);
  plan->off_Wp = off;
  off += align256((size_t)plan->V_pad * plan->hS * (tbytes == 4 ? SliceK<float>::value : SliceK<bf16_t>::value) * tbytes);
  plan->off_flag = plan->off_idx = plan->off_inv = plan->off_nact = 0;
  if (active) {
    plan->off_flag = off;
    off += align256((size_t)N * 4);
    plan->off_idx = off;
    off += align256((size_t)N * 4);
    plan->off_inv = off;
    off += align256((size_t)N * 4);
    plan->off_nact = off;  // [0] count, [1..2] parameter flags
    off += 256;
  }
  plan->ws_bytes = off;
  return true;
}

hipError_t fwd_launch(int dtype, const FwdPlan& plan, FwdParams p, char* ws, float* O, float* lse, float* m_out,
                      float* l_out, hipStream_t stream) {
  if (p.N == 0) return hipSuccess;
  p.n_tb = plan.n_tb;
  p.n_split = plan.n_split;
  p.n_vt = plan.n_vt;
  p.part_m = reinterpret_cast<float*>(ws + plan.off_m);
  p.part_l = reinterpret_cast<float*>(ws + plan.off_l);
  p.part_acc = reinterpret_cast<float*>(ws + plan.off_acc);
  p.Ep = ws + plan.off_Ep;
  p.biasp = reinterpret_cast<const float*>(ws + plan.off_bias);
  p.hp = ws + plan.off_hp;
  p.Wp = ws + plan.off_Wp;
  p.hS = plan.hS;
  hipError_t e;
  switch (dtype) {
    case kBF16: e = pack<bf16_t>(p, plan, stream); break;
    case kF16: e = pack<f16_t>(p, plan, stream); break;
    case kF32: e = pack<float>(p, plan, stream); break;
    case kFP8: e = pack<bf16_t>(p, plan, stream); break;
    default: return hipErrorInvalidValue;
  }
  if (e != hipSuccess) return e;
  // one pass per slice of E's columns (one pass unless D exceeds the slice width)
  const int64_t esz = dtype == kF32 ? 4 : 2;
  const int D = p.D;
  for (int d0 = 0; d0 < (D > 0 ? D : 1); d0 += plan.DS) {
    FwdParams q = p;
    q.E = static_cast<const char*>(p.E) + d0 * esz;
    q.D = D - d0 < plan.DS ? D - d0 : plan.DS;
    switch (dtype) {
      case kBF16: e = pack_et<bf16_t>(q, plan, stream); if (e == hipSuccess) e = dispatch_dp<bf16_t>(plan, q, stream); break;
      case kF16: e = pack_et<f16_t>(q, plan, stream); if (e == hipSuccess) e = dispatch_dp<f16_t>(plan, q, stream); break;
      case kF32: e = pack_et<float>(q, plan, stream); if (e == hipSuccess) e = dispatch_dp<float>(plan, q, stream); break;
      default: e = pack_et<bf16_t>(q, plan, stream); if (e == hipSuccess) e = dispatch_dp_f8(plan, q, stream); break;
    }
    if (e != hipSuccess) return e;
    // every pass computes the same scores, so each writes the same lse (m, l); O gets its columns
    timing_begin(kKindFwdCombine, stream);
    const int64_t n_threads = (int64_t)p.N * (q.D > 0 ? q.D : 1);
    fwd_combine_kernel<<<(int)((n_threads + 255) / 256), 256, 0, stream>>>(
        p.part_m, p.part_l, p.part_acc, plan.n_part, p.N, q.D, (int64_t)plan.DP * p.N, p.N, 1, O ? O + d0 : nullptr,
        D, lse, m_out, l_out);
    timing_end(kKindFwdCombine, stream);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  return hipSuccess;
}

namespace {

// Everything of the active-token forward before its passes: the parameter flags (bad[0..1], set
// while W is packed and by the E / bias scan), the per-token flags and their compaction into
// positions (idx, inv, n_act[0]), the device-side token blocks and splits (n_act[3..4]), and the
// active tokens' h rows packed in position order.  n_act points at the count block:
// [0] count, [1..2] parameter flags, [3..4] token blocks and splits.
template <class T>
hipError_t active_setup(const FwdPlan& plan, const FwdParams& p, const float* weight, int* flag, int* idx, int* inv,
                        int* n_act, int* bad, hipStream_t stream) {
  timing_begin(kKindPack, stream);
  const bool scale_bad = !std::isfinite(p.scale);
  fwd_flags_init_kernel<<<1, 64, 0, stream>>>(bad, scale_bad ? 1 : 0, (p.bias || p.V == 0) ? 1 : 0);
  hipError_t e = hipGetLastError();
  // W once (as fwd_launch packs it), checked for non-finite values on the way
  PackExtra wx;
  wx.nonfinite = bad;
  T* const Wp = const_cast<T*>(static_cast<const T*>(p.Wp));
  if (e == hipSuccess) e = pack_src<T>(p.W, p.w_f32, p.ldw, p.V, p.K, plan.hS, plan.V_pad, Wp, stream, nullptr, wx);
  const int64_t work = (int64_t)p.V * (p.D > 0 ? p.D : 1);
  if (e == hipSuccess && work > 0 && (p.D > 0 || p.bias)) {
    const int blocks = (int)((work + 255) / 256 < 2048 ? (work + 255) / 256 : 2048);
    fwd_param_scan_kernel<T><<<blocks, 256, 0, stream>>>(static_cast<const T*>(p.E), p.lde, p.V, p.D, p.bias, bad);
    e = hipGetLastError();
  }
  if (e == hipSuccess) {
    const unsigned blocks = (unsigned)((p.N + 3) / 4);
    if (sizeof(T) == 2 && p.h_f32)
      fwd_active_flag_kernel<float, T><<<blocks, 256, 0, stream>>>(weight, static_cast<const float*>(p.h), p.ldh,
                                                                   p.N, p.K, bad, flag);
    else
      fwd_active_flag_kernel<T, T><<<blocks, 256, 0, stream>>>(weight, static_cast<const T*>(p.h), p.ldh, p.N, p.K,
                                                               bad, flag);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = compact_tokens(flag, p.N, idx, inv, n_act, stream);
  if (e == hipSuccess) {
    fwd_active_grid_kernel<<<1, 64, 0, stream>>>(n_act, plan.BM, plan.n_tb, plan.n_split, plan.n_vt);
    e = hipGetLastError();
  }
  // h rows of the active tokens in position order, zeros past them
  PackExtra hx;
  hx.rows = idx;
  hx.n_rows = n_act;
  T* const hp = const_cast<T*>(static_cast<const T*>(p.hp));
  if (e == hipSuccess) e = pack_src<T>(p.h, p.h_f32, p.ldh, p.N, p.K, plan.hS, plan.N_pad, hp, stream, nullptr, hx);
  timing_end(kKindPack, stream);
  return e;
}

}  // namespace

hipError_t fwd_launch_active(int dtype, const FwdPlan& plan, FwdParams p, const float* weight, char* ws, float* O,
                             float* lse, hipStream_t stream) {
  if (p.N == 0) return hipSuccess;
  if (!plan.active || dtype == kFP8) return hipErrorInvalidValue;
  p.n_tb = plan.n_tb;
  p.n_split = plan.n_split;
  p.n_vt = plan.n_vt;
  p.part_m = reinterpret_cast<float*>(ws + plan.off_m);
  p.part_l = reinterpret_cast<float*>(ws + plan.off_l);
  p.part_acc = reinterpret_cast<float*>(ws + plan.off_acc);
  p.Ep = ws + plan.off_Ep;
  p.biasp = reinterpret_cast<const float*>(ws + plan.off_bias);
  p.hp = ws + plan.off_hp;
  p.Wp = ws + plan.off_Wp;
  p.hS = plan.hS;
  int* flag = reinterpret_cast<int*>(ws + plan.off_flag);
  int* idx = reinterpret_cast<int*>(ws + plan.off_idx);
  int* inv = reinterpret_cast<int*>(ws + plan.off_inv);
  int* n_act = reinterpret_cast<int*>(ws + plan.off_nact);
  p.n_act = n_act;
  hipError_t e;
  switch (dtype) {
    case kBF16: e = active_setup<bf16_t>(plan, p, weight, flag, idx, inv, n_act, n_act + 1, stream); break;
    case kF16: e = active_setup<f16_t>(plan, p, weight, flag, idx, inv, n_act, n_act + 1, stream); break;
    case kF32: e = active_setup<float>(plan, p, weight, flag, idx, inv, n_act, n_act + 1, stream); break;
    default: return hipErrorInvalidValue;
  }
  if (e != hipSuccess) return e;
  const int64_t esz = dtype == kF32 ? 4 : 2;
  const int D = p.D;
  for (int d0 = 0; d0 < (D > 0 ? D : 1); d0 += plan.DS) {
    FwdParams q = p;
    q.E = static_cast<const char*>(p.E) + d0 * esz;
    q.D = D - d0 < plan.DS ? D - d0 : plan.DS;
    switch (dtype) {
      case kBF16: e = pack_et<bf16_t>(q, plan, stream); if (e == hipSuccess) e = dispatch_dp<bf16_t>(plan, q, stream); break;
      case kF16: e = pack_et<f16_t>(q, plan, stream); if (e == hipSuccess) e = dispatch_dp<f16_t>(plan, q, stream); break;
      default: e = pack_et<float>(q, plan, stream); if (e == hipSuccess) e = dispatch_dp<float>(plan, q, stream); break;
    }
    if (e != hipSuccess) return e;
    timing_begin(kKindFwdCombine, stream);
    const int64_t n_threads = (int64_t)p.N * (q.D > 0 ? q.D : 1);
    fwd_combine_active_kernel<<<(int)((n_threads + 255) / 256), 256, 0, stream>>>(
        p.part_m, p.part_l, p.part_acc, inv, n_act, plan.BM, plan.WV, p.N, q.D, plan.DP, O + d0, D, lse);
    timing_end(kKindFwdCombine, stream);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t shard_combine(int S, int N, int D, const float* m, const float* l, const float* acc, float* O, float* lse,
                         hipStream_t stream) {
  const int64_t n_threads = (int64_t)N * (D > 0 ? D : 1);
  if (n_threads == 0) return hipSuccess;
  timing_begin(kKindFwdCombine, stream);
  fwd_combine_kernel<<<(int)((n_threads + 255) / 256), 256, 0, stream>>>(m, l, acc, S, N, D, (int64_t)N * D, 1, D, O,
                                                                         D, lse, nullptr, nullptr);
  timing_end(kKindFwdCombine, stream);
  return hipGetLastError();
}

}  // namespace swvr
