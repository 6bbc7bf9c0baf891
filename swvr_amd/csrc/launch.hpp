// Host-side interface between the C ABI (abi.hip) and the kernel files.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace swvr {

// Kernel kinds, for the launch timing record.
enum KernelKind {
  kKindFwdTile = 0,
  kKindFwdCombine,
  kKindBwdDelta,
  kKindBwdScores,
  kKindBwdGemm,
  kKindBwdReduce,
  kKindFill,
  kKindPack,
  kKindBwdExpand,
  kKindLoss,
  kKindQuant,
  kKindF64,
  kKindProbe,
  kNumKinds
};

// Timing hooks (abi.hip): bracket one launch when timing is enabled.
void timing_begin(int kind, hipStream_t stream);
void timing_end(int kind, hipStream_t stream);

// ---------------------------------------------------------------- forward
struct FwdParams {
  const void* h;
  int64_t ldh;
  const void* W;
  int64_t ldw;
  const void* E;
  int64_t lde;
  const float* bias;  // fp32 [V] or null
  float scale;
  int N, K, V, D;
  int n_tb, n_split, n_vt;
  float* part_m;       // [n_part][N]
  float* part_l;       // [n_part][N]
  float* part_acc;     // [n_part][DP][N]
  const void* Ep;      // packed E^T tiles [n_vt][DP][BV], compute dtype
  const float* biasp;  // packed bias [V_pad], -inf past V
  const void* hp;      // h packed in its tiles' LDS image (pack_rows_tiled_kernel)
  const void* Wp;      // W packed the same way, [V_pad] rows
  int hS;              // reduction slices of both
  int h_f32, w_f32;    // h / W stored in fp32 (rounded to the compute dtype as they are packed)
  const float* h_scale;  // e4m3 forward: [1] dequantisation scale of h, else null
  const float* w_scale;  // e4m3 forward: [V] dequantisation scales of W's rows, else null
  // Active-token forward: [0] the count of active tokens, whose rows are packed
  // in position order (hp), [3] / [4] the token blocks and vocabulary splits
  // (active_grid), all on the device; null: every token, at its own row.
  const int* n_act;
};

// Token blocks and vocabulary splits of an active-token forward, from the
// device count of active tokens.  The launch has grid = n_tb_max x n_split0
// workgroups (the all-token tiling: whole rounds of kFwdRound, one workgroup
// per CU); with n_act active tokens the first n_tb x n_split of them work.  The
// split count minimises the forward's duration in the round model, rounds x
// vocabulary tiles per workgroup ~ ceil(n_tb x s / kFwdRound) / s, over
// s = n_split0 .. min(n_vt / 2, 2 x grid / n_tb) (the smallest such s on a
// tie): the partial buffers hold 2 x grid workgroups' partials.  Computed once
// per call (fwd_active_grid_kernel) into the count's block, so every kernel of
// the forward uses the same values and the host needs no copy of them.
constexpr int kFwdRound = 256;
__host__ __device__ inline void active_grid(int n_act, int BM, int n_tb_max, int n_split0, int n_vt, int* n_tb,
                                            int* n_split) {
  int tb = n_act <= 0 ? 0 : (n_act + BM - 1) / BM;
  if (tb > n_tb_max) tb = n_tb_max;
  int sp = n_split0;
  if (tb > 0) {
    const int cap = n_vt / 2 > 1 ? n_vt / 2 : 1;
    const int64_t fit = 2 * (int64_t)n_tb_max * n_split0 / tb;
    const int hi = fit < cap ? (int)fit : cap;
    int64_t best_r = ((int64_t)tb * sp + kFwdRound - 1) / kFwdRound;
    for (int s = n_split0 + 1; s <= hi; ++s) {
      const int64_t r = ((int64_t)tb * s + kFwdRound - 1) / kFwdRound;
      if (r * sp < best_r * s) {  // r / s < best_r / sp
        best_r = r;
        sp = s;
      }
    }
  }
  *n_tb = tb;
  *n_split = sp;
}

struct FwdPlan {
  int BV, BM, DP;
  int DS, n_dslices;     // embedding columns per pass, passes (D > DS runs in slices of E's columns)
  int n_tb, n_vt, n_split, n_part;
  int V_pad;
  int64_t N_pad;         // token rows of the packed h
  int hS;                // reduction slices of the packed h and W
  size_t off_m, off_l, off_acc, off_Ep, off_bias, off_hp, off_Wp, ws_bytes;
  // active-token forward: per-token flags, positions, the count and the
  // non-finite parameter flag (ws_bytes includes them only when planned so)
  bool active;
  int WV;
  size_t off_flag, off_idx, off_inv, off_nact;
};

// fwd_plan / fwd_launch dtype of the e4m3 forward (h, W in e4m3; E in bf16).
constexpr int kFwdFP8 = 3;

// Tile shape, split count and workspace for a forward call; ok=false if the
// dtype / D combination is unsupported.
bool fwd_plan(int dtype, int64_t N, int64_t K, int64_t V, int64_t D, FwdPlan* plan, bool active = false);
// O / lse, or with m_out / l_out set the merged partial softmax (m, l, and the
// unnormalised acc in O) of the vocabulary rows given.
hipError_t fwd_launch(int dtype, const FwdPlan& plan, FwdParams p, char* ws, float* O, float* lse, float* m_out,
                      float* l_out, hipStream_t stream);
// The forward of the tokens with a non-zero weight (weight: fp32 [N]); O rows
// and lse of the others are 0.  A zero-weight token whose h row holds an
// infinity or a NaN stays active, and so does every token when W, E or the
// bias holds a NaN or +inf or when every bias entry is -inf: the rows whose
// loss the reference makes NaN (0 * NaN) are computed.  Plan with active set.
hipError_t fwd_launch_active(int dtype, const FwdPlan& plan, FwdParams p, const float* weight, char* ws, float* O,
                             float* lse, hipStream_t stream);
// Order-preserving compaction of flagged tokens (flag[n] != 0): idx[q] = token
// of position q, inv[n] = position of token n or -1, n_act[0] = count.
hipError_t compact_tokens(const int* flag, int N, int* idx, int* inv, int* n_act, hipStream_t stream);
// Merge S vocabulary shards' partials (m, l: [S][N]; acc: [S][N][D]) in shard order.
hipError_t shard_combine(int S, int N, int D, const float* m, const float* l, const float* acc, float* O, float* lse,
                         hipStream_t stream);

// ---------------------------------------------------------------- backward
struct BwdPlan {
  int DP;
  int BM, BV;            // dS kernel tile: BM tokens x BV vocabulary
  int GM, GN;            // gradient GEMM tile
  int n_tb;              // token blocks of the dS kernel
  int64_t N_pad;         // token stride of the dS stage
  int64_t C;             // vocabulary rows per chunk (multiple of BV)
  int n_chunks;
  int G;                 // token groups of the dS kernel (a full chunk)
  int wgs;               // workgroups the dS kernel's tiling fills the chip with (G per chunk from it)
  int n_gpart;           // dE / db partials per chunk
  int kind;              // scores kernel: kScoresGeneral, kScoresRing (narrow), kScoresWide
  bool dh_acc;           // dh accumulates in fp32 (over the active tokens), then expands into gh
  int V_pad;             // vocabulary rows of the packed E / bias
  int hS;                // reduction slices of the packed h and W
  size_t off_stage, off_pe, off_pb, off_dh, off_gO, off_gOt, off_lsed, off_Ep, off_bias, off_hp, off_Wp;
  size_t off_flag, off_idx, off_inv, off_nact, off_delta, off_hc, off_Wc, ws_bytes;
  int hS8;               // e4m3 scores: reduction slices of the packed e4m3 h and W (K8 / 2 pairs)
  size_t off_hqc, off_mult;
  size_t off_pstage;     // P stage (wide scores kernel), the dS stage's layout
};

// Scores kernels of the backward (BwdPlan::kind).
enum { kScoresGeneral = 0, kScoresRing = 1, kScoresWide = 2 };
// With the wide scores kernel, dE^T = gO^T P is formed by the gradient GEMM launch as up to this
// many partial sums over equal runs of the positions (fixed-order sum after the launch): one run
// per 2048 token rows (64 reduction slices), 1 to kDeSplit (de_split).
constexpr int kDeSplit = 8;
inline int de_split(int64_t n_pad) {
  const int64_t s = n_pad / 2048;
  return s < 1 ? 1 : s > kDeSplit ? kDeSplit : (int)s;
}

// w_f32: W is stored in fp32 and needs a row-major copy in the compute dtype
// (the dh product reads W rows directly).
// K8 > 0: the scores are recomputed from e4m3 h and W of K8 bytes per row.
bool bwd_plan(int dtype, int64_t N, int64_t K, int64_t V, int64_t D, int64_t chunk, bool need_gh,
              BwdPlan* plan, bool w_f32 = false, int64_t K8 = 0);

struct BwdParams {
  const void* h;
  int64_t ldh;
  const void* W;
  int64_t ldw;
  const void* E;
  int64_t lde;
  const float* bias;
  float scale;
  int N, K, V, D;
  const float* O;
  const float* lse;
  const float* gO;
  const float* glse;
  void* gh;
  int gh_dtype;
  void* gW;
  int gW_dtype;
  void* gE;
  int gE_dtype;
  float* gb;
  char* ws;
  int h_f32, w_f32;    // h / W stored in fp32 (rounded to the compute dtype as they are read)
  // e4m3 scores (null hq: the compute dtype's): h and W as e4m3 bytes, K8 per
  // row, leading dims in bytes, with the forward's dequantisation scales
  const void* hq;
  int64_t ldhq;
  const void* Wq;
  int64_t ldwq;
  const float* h_scale;
  const float* w_scale;
  int K8;
};

hipError_t bwd_launch(int dtype, const BwdPlan& plan, const BwdParams& p, hipStream_t stream);

// ---------------------------------------------------------------- MSE loss
struct MseParams {
  const float* O;       // [N][D] fp32
  const float* lse;     // [N] fp32
  const void* target;   // [N][ldt], target_dtype (0 bf16, 1 f16, 2 f32)
  int64_t ldt;
  int target_dtype;
  const float* weight;  // [N] fp32 or null
  int N, D;
  float z;              // z-loss weight
  int reduce;           // 0 none, 1 sum, 2 mean
  float* per_tok;       // [N] (reduce == 0) or null
  float* out;           // [1] (reduce != 0)
  float* scale;         // [1] (reduce != 0): the c of the loss
  float* gO;            // [N][D] or null
  float* glse;          // [N] or null (with gO)
};
size_t mse_workspace_bytes(int N);
// Largest N of the allocation-free loss entry point, whose partial sums live in
// a fixed device array (loss.hip) instead of the caller's workspace.
constexpr int kMseNoAllocMaxTokens = 1 << 22;
// Address of that array on the device of `stream` (the current device for the
// null stream), looked up once per device.
hipError_t mse_noalloc_scratch(hipStream_t stream, void** ptr);

// ---------------------------------------------------------------- e4m3 quantisation
struct QuantParams {
  const void* x;   // [R][ld], x_dtype (0 bf16, 1 f16, 2 f32)
  int64_t ld;
  int x_dtype;
  int R, K, Kp;    // rows, columns, output columns (zero past K)
  int per_row;     // scales per row ([R]) or one for the matrix ([1])
  void* out;       // e4m3 bytes [R][ldo]
  int64_t ldo;
  float* scale;
  float* amax;     // per-tensor: [R] row amaxes (workspace)
};
hipError_t quant_launch(const QuantParams& q, hipStream_t stream);

// ---------------------------------------------------------------- fp64
struct F64Params {
  const double* h;
  int64_t ldh;
  const double* W;
  int64_t ldw;
  const double* E;
  int64_t lde;
  const double* bias;  // [V] or null
  double scale;
  int N, K, V, D;
  int64_t chunk;
  double* O;            // forward: [N][D]; backward: the forward's O (read)
  double* lse;          // forward: [N]; backward: the forward's lse (read)
  const double* gO;     // backward: [N][D]
  const double* glse;   // backward: [N]
  double* gh;           // [N][K] or null
  double* gW;           // [V][K] or null
  double* gE;           // [V][D] or null
  double* gb;           // [V] or null
  char* ws;
};
// Vocabulary rows per chunk and workspace bytes of the fp64 forward / backward.
void f64_plan(int64_t N, int64_t V, int64_t D, int64_t chunk, int64_t* C, size_t* fwd_bytes, size_t* bwd_bytes);
hipError_t f64_fwd(const F64Params& p, hipStream_t stream);
hipError_t f64_bwd(const F64Params& p, hipStream_t stream);

// Matrix-core throughput probe (probe.hip): workgroups of 8 waves, iters k16 steps of
// 8 MFMAs per wave; out receives workgroups * 512 floats.
hipError_t probe_mfma(int workgroups, int iters, int mode, float* out, hipStream_t stream);
hipError_t mse_launch(const MseParams& p, void* ws, hipStream_t stream);

}  // namespace swvr
