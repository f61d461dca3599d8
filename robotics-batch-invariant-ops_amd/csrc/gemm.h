// Host-side interface of the batched GEMM launcher shared by the GEMM, attention and MoE entry
// points.
#pragma once

#include "gemm_core.h"

namespace biops {

enum { kEpiPlain = 0, kEpiBias = 1, kEpiSwiglu = 2 };

// One launch covers nb1*nb2 independent GEMMs C[b] = A[b] . B[b] of equal shape.
// Batch b = b1*nb2 + b2 addresses X + b1*sX1 + (b2/gX)*sX2 (gA = gC = 1, gB = args.gB).
// B is K-major (column n at B + n*ldb, K contiguous) or N-major (K row k at B + k*ldb).
// In SwiGLU mode B holds the gate weights and B2 the up weights (same layout and strides) and
// N counts output columns (each needs one gate and one up column).
//
// Grouped rows (grp != nullptr, nb1 = nb2 = 1): the rows of A and C are split into row groups
// g, each multiplied by its own B + g*sB1.  The device table grp holds
//   grp[0]                      number of m-tiles J,
//   grp[4 + 4j .. 4 + 4j + 2]   {group, first row, end row of the group} of m-tile j,
// with m-tiles BM rows high (the BM that grouped_tile_rows() returns for the same problem; a
// group's last m-tile is cut at the group's end row).  grp_rows bounds the rows of all groups
// together and grp_groups the number of non-empty groups; the launch is sized for the worst
// case J <= cdiv(grp_rows, BM) + min(grp_groups, grp_rows) and the tiles past J do nothing.
struct BmmArgs {
  const void* A;
  const void* B;
  const void* B2;
  void* C;
  const void* bias;
  int64_t M, N, K;
  int64_t lda, ldb, ldc;
  int64_t nb1, nb2, gB;
  int64_t sA1, sA2, sB1, sB2, sC1, sC2;
  const int32_t* grp;
  int64_t grp_rows, grp_groups;
  // Grouped rows only: row p of the packed problem reads A row a_rows[p] (nullptr: row p).
  const int32_t* a_rows;
  // filled by the launcher
  int64_t tiles_m, tiles_n, total;
  int32_t a_vec, b_vec, c_vec;
  int32_t nt_store;  // four-wave entries: whole tiles store with non-temporal stores
};

constexpr int kGrpHeader = 4;
constexpr int kGrpStride = 4;
// Smallest m-tile height grouped_tile_rows() returns (tables of grouped launches are sized for it).
constexpr int kMinGroupedTileRows = 16;

int launch_bmm(int dtype, BmmArgs a, int epi, bool b_kmajor, hipStream_t stream);

// Tile height of the entry launch_bmm picks for a grouped problem whose M is the mean group
// size (0 on error).
int grouped_tile_rows(int dtype, BmmArgs a, int epi, bool b_kmajor);

// Tail m-tiles of a grouped problem: when the entry launch_bmm picks has m-tiles of 128 rows or
// more, the groups hold at least two such m-tiles on average and B is a 16-bit N-major matrix
// on the direct path, a group's last m-tile with fewer rows than the returned count is better
// run apart, on the weight-streaming tile (one such sliver in a 256-row tile costs a whole
// tile); 0 when the problem has no such split.
int grouped_tail_rows(int dtype, BmmArgs a, int epi, bool b_kmajor);
// The tail m-tiles listed in a.grp (m-tiles of up to grouped_tail_rows() rows) on the
// weight-streaming tile; same bits as any other entry.
int launch_grouped_tail(int dtype, BmmArgs a, int epi, hipStream_t stream);

// Packed variable-length attention work list (host and device copies share the layout):
//   plan[0] items, plan[1] QK^T tiles, plan[2] PV tiles, plan[3] score rows,
//   plan[4] score elements, plan[5..7] reserved,
//   plan[8 + 8*i ..] = {q_start, q_len, kv_start, kv_len, s_off, qk_tile0, pv_tile0, row0}
// for every sequence i with q_len > 0 and kv_len > 0.  The tile counts are for the fixed
// varlen tile kVarlenBM x kVarlenBN; every head of a sequence is a separate GEMM problem.
constexpr int kPlanHeader = 8;
constexpr int kPlanStride = 8;
constexpr int kVarlenBM = 128;
constexpr int kVarlenBN = 128;

enum { kGroupQK = 0, kGroupPV = 1 };

// Score rows of a varlen sequence are stored at a pitch rounded up to 8 elements so that every
// row starts 16-byte aligned (vector loads in the softmax and the PV GEMM).
__host__ __device__ __forceinline__ int64_t varlen_score_ld(int64_t kv_len) { return (kv_len + 7) & ~int64_t(7); }

// Grouped GEMM over the plan: QK mode S_i,h = Q_i,h . K_i,h'^T; PV mode O_i,h = P_i,h . V_i,h'
// (h' = h / group).  Token strides s*_t and head strides s*_h are in elements.
struct GroupedArgs {
  const void* q; const void* k; const void* v; void* s; void* out;
  const int64_t* plan;
  int64_t items, total_tiles, heads, group, d, dv;
  int64_t sq_t, sq_h, sk_t, sk_h, sv_t, sv_h, so_t, so_h;
};

int launch_grouped(int dtype, const GroupedArgs& a, int mode, hipStream_t stream);

// Resolve the B operand layout from its (K, N) strides; false if neither is unit-stride.
bool b_layout(int64_t K, int64_t N, int64_t sBk, int64_t sBn, bool& kmajor, int64_t& ldb);

}  // namespace biops
