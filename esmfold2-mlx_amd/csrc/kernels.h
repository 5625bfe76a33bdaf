// Internal launch interface between the C ABI (capi.cpp) and the kernels.
// Arguments are validated by the caller before any launcher runs.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace esm {

typedef _Float16 half_t;

struct ProjectArgs {
  const half_t* z;      // [B, L, L, C]
  const half_t* mask;   // [B, L, L] or nullptr
  const float* ln_w;    // [C]
  const float* ln_b;    // [C]
  float eps;
  const half_t* w;      // [4c, C]
  half_t* a;            // [B, c, L, ld]
  half_t* b;            // [B, c, L, ld]
  int B, L, ld;
  int transpose;        // 1: store cell (r, s) at row s, column r
  int ntiles, tiles_per_line;
  // frag = 1: a and b in MFMA-fragment order instead of [B, c, L, ld] (see FragLayout),
  // with tiles of 8 x 8 cells (tiles_per_line = tiles per dimension)
  int frag, rbn, kbn;
};

// The MFMA-fragment layout of a contraction operand (kernel (a) writes it for the fused
// forward, kernel (b) reads it): plane p = b * c + channel holds rbn x kbn tiles of 32 rows
// by 16 k, rbn = ceil(L / 32), kbn = ceil(L / 16); a tile is 64 lanes x 8 halfs, lane l
// holding row 32 rb + l % 32, k = 16 kb + 8 (l / 32) .. +7, i.e. exactly the operand of one
// v_mfma_f32_32x32x16_f16, so the contraction loads each operand fragment with one fully
// coalesced 1 KB read. Rows at or past L are never read; k at or past L is zero.
struct FragLayout {
  static constexpr int kTileHalfs = 64 * 8;
  static size_t plane_halfs(int L) { return (size_t)((L + 31) / 32) * ((L + 15) / 16) * kTileHalfs; }
};

struct ContractArgs {
  const half_t* a;      // [batch, L, ld], or (frag) [batch] planes of FragLayout
  const half_t* b;      // [batch, L, ld], or (frag) [batch] planes of FragLayout
  half_t* x;            // [batch, L, ldx]
  int batch, L, ld, ldx;
  float scale;
  int frag;             // operands in FragLayout
};

struct EpilogueArgs {
  const half_t* x;      // [B, c, L, ldx]
  int ldx;
  const half_t* z;      // [B, L, L, C]
  const half_t* mask;   // [B, L, L] or nullptr
  const float* ln_in_w;
  const float* ln_in_b;
  float eps_in;
  const float* ln_mix_w;
  const float* ln_mix_b;
  float eps_mix;
  const half_t* w_emit; // [C, c]
  const half_t* w_gate; // [C, C]
  half_t* out;          // [B, L, L, C]
  int B, L;
  int residual, out_mask;
  int ntiles, tiles_per_line;
};

struct Q8Args {
  const half_t* x;      // [M, K]
  const uint8_t* q;     // [N, K]
  const half_t* s;      // [N, K/64]
  const half_t* b;      // [N, K/64]
  half_t* y;            // [M, N]
  int M, K, N;
  int mtiles, ntiles;   // tiles of kQ8TileM x (32 nb) outputs
  int splits;           // K ranges per tile
  float* part;          // [splits, M, N] fp32 partials, or nullptr: y written directly (splits 1)
  const uint32_t* sb;   // packed scales [N/32, K/64, 32] (b << 16 | s), or nullptr
  const uint8_t* qp;    // codes packed by q8_pack_codes (needs sb), or nullptr: q is read
  int swiglu;           // weight rows in SwiGLU pairs (each 160-row tile: 80 gate rows, then the
                        // matching 80 up rows): y [M, N/2] = silu(gate) * up instead of [M, N]
  int nb;               // 32-row weight blocks per tile: kQ8TileNbNarrow or kQ8TileNbWide
};

// q8 GEMM tile: kQ8TileM rows of x by 32 nb weight rows (nb = 4 or 5, chosen per call by the
// launch plan), kQ8Waves waves per workgroup. The packed layouts do not depend on nb.
constexpr int kQ8TileM = 64;
constexpr int kQ8TileNbNarrow = 4;
constexpr int kQ8TileNbWide = 5;
constexpr int kQ8Waves = 4;
// Bytes of the device scratch q8_linear_noalloc keeps its split-K partials in.
constexpr size_t kQ8ScratchBytes = (size_t)16 << 20;
// The device address of that scratch on the current device (taken once per device).
hipError_t q8_scratch_address(float** ptr);

struct TransitionArgs {
  const half_t* z;      // [cells, C]
  half_t* out;          // [cells, C], may be z
  const float* ln_w;    // [C]
  const float* ln_b;    // [C]
  float eps;
  const half_t* w1;     // [H, C]
  const half_t* w2;     // [H, C] (SwiGLU) or nullptr (ReLU)
  const half_t* w3;     // [C, H]
  size_t ncells;
  int ntiles, H;
};

struct EsmcLnArgs {
  const float* x;       // [M, D] fp32 residual
  const half_t* y;      // [M, D] or nullptr: x_out = x + alpha * y
  const float* yp;      // [splits, M, D] fp32 split-K partials of y, or nullptr: y = fp16(sum in split order)
  int splits;
  float alpha;
  float* x_out;         // [M, D] (may be x; unused without y)
  const float* w;       // [D]
  const float* b;       // [D] or nullptr
  float eps;
  half_t* h;            // [M, D] LN output (fp16), or nullptr
  float* h32;           // [M, D] LN output (fp32), or nullptr
  int M, D;
};

struct EsmcRopeArgs {
  const half_t* qkv;    // [B*L, 3D]
  const float* q_ln;    // [D]
  const float* k_ln;    // [D]
  float eps;
  half_t* q;            // [B, H, L, 64]
  half_t* k;
  half_t* v;
  int B, L, H;
  float log2_base;
};

struct EsmcAttnArgs {
  const half_t* q;      // [B, H, L, 64]
  const half_t* k;
  const half_t* v;
  const int* sid;       // [B, L] chain ids or nullptr
  half_t* o;            // [B, L, H*64]
  int B, L, H;
  float scale_log2;     // scale * log2(e)
};

struct ParcaeArgs {
  const float* z;         // [cells, C] recurrent state
  const float* z_init;    // [cells, C]
  const float* refined;   // [cells, C] (the LM encoder's output)
  const float* ln_w;      // [C]
  const float* ln_b;      // [C]
  float eps;
  const float* a;         // [C]
  const half_t* b_mat;    // [C, C] (out, in)
  float* z_out;           // [cells, C], may be z
  size_t ncells;
  int ntiles;
  int C;                  // 128 or 256
};

struct DistoArgs {
  const float* r;         // [B, L, L, C]
  const half_t* w;        // [nbins, C]
  const float* bias;      // [nbins]
  const float* centers;   // [nbins]
  float* ed;              // [B, L, L]
  int B, L, nbins;
  int C;                  // 128 or 256
};

// Wide path (pair widths other than 128): epilogues of wide_gemm.
enum : int { kWideGateCM = 0, kWideResGate = 1, kWideRelu = 2, kWideSwiglu = 3, kWideResid = 4 };

struct WideArgs {
  const half_t* a1;     // [cells, K] fp16 rows (the A operand of GEMM 1)
  const half_t* a2;     // [cells, K] (GEMM 2's A; nullptr or a1: the same operand)
  const half_t* w1;     // [N, K]
  const half_t* w2;     // [N, K] or nullptr (single GEMM)
  int K, N;
  int B, L;             // cells = B * L * L, tiled along lines of L cells
  int tiles_per_line;   // ceil(L / 128)
  int transpose;        // 1: line = column, positions along rows (the incoming operands)
  int frag;             // GATE_CM with K <= 256: a, b planes in FragLayout, tiles of 8 x 8 cells
  int rbn, kbn;         // FragLayout tiles per plane (frag)
  half_t* out;          // [cells, ldo] cell-major output (all but GATE_CM)
  int ldo;
  const half_t* z;      // [cells, ldo] residual (RESGATE with residual, RESID)
  int residual;         // RESGATE: add z
  const half_t* mask;   // [cells] or nullptr (GATE_CM; RESGATE with out_mask)
  int out_mask;
  half_t* plane_a;      // GATE_CM: outputs [0, c) -> a, [c, 2c) -> b, [B, c, L, ld] channel-major
  half_t* plane_b;
  int c, ld;
};

// Cells per tile of the per-cell kernels (a) and (c).
constexpr int kCellTile = 64;
// Cells per unit of the epilogue kernel (c): one 32-column MFMA tile of one pair row;
// waves per epilogue workgroup (two per SIMD).
constexpr int kEpiUnit = 32;
constexpr int kEpiWaves = 8;

// Each launcher returns the hipError_t of the launch.
hipError_t launch_project(const ProjectArgs& a, int grid, hipStream_t s);
hipError_t launch_contract(const ContractArgs& a, hipStream_t s);
hipError_t launch_epilogue(const EpilogueArgs& a, int grid, hipStream_t s);
hipError_t launch_q8_linear(const Q8Args& a, hipStream_t s);
// SwiGLU pair rows: weight row of output column c of a [M, N] product in the pair order,
// gate f <-> column 160 (f / 80) + f % 80, up f <-> that + 80 (N a multiple of 160).
constexpr int kQ8SwigluHalf = 80;
hipError_t launch_transition(const TransitionArgs& a, int grid, hipStream_t s);
hipError_t launch_esmc_ln(const EsmcLnArgs& a, hipStream_t s);
hipError_t launch_parcae_step(const ParcaeArgs& a, int grid, hipStream_t s);
hipError_t launch_expected_distance(const DistoArgs& a, int grid, hipStream_t s);
hipError_t launch_abs_diff_quantile(const float* x, const float* y, size_t n, float q, float* out, hipStream_t s);
hipError_t launch_esmc_qk_rope(const EsmcRopeArgs& a, hipStream_t s);
hipError_t launch_esmc_attention(const EsmcAttnArgs& a, hipStream_t s);
hipError_t launch_esmc_swiglu(const half_t* x12, half_t* y, size_t M, int F, hipStream_t s);
hipError_t launch_q8_pack(const half_t* s, const half_t* b, uint32_t* sb, int N, int K, hipStream_t st);
// Bytes of q8_pack_codes' layout: per 32-row block and step of two groups, 4 waves x 64
// lanes x 16 bytes.
constexpr size_t q8_packed_codes_size(int N, int K) {
  return (size_t)((N + 31) / 32) * (size_t)((K / 64 + 1) / 2) * (size_t)(kQ8Waves * 1024);
}
// Words of q8_pack_scales' layout: per 32-row block and group, 32 words b << 16 | s.
constexpr size_t q8_packed_scales_words(int N, int K) { return (size_t)((N + 31) / 32) * (size_t)(K / 64) * 32; }
hipError_t launch_q8_pack_codes(const uint8_t* q, uint8_t* qp, int N, int K, hipStream_t st);
hipError_t launch_ln_rows(const void* x, const float* x2, bool in_f32, const float* w, const float* b, float eps,
                          half_t* out, size_t rows, int C, hipStream_t s);
hipError_t launch_ln_cf_to_cl(const half_t* x, int ldx, const float* w, const float* b, float eps, half_t* y, int B,
                              int L, int c, hipStream_t s);
long long wide_gemm_blocks(const WideArgs& a);
// cus > 0 with K = 128 or 256: the weight-stationary persistent form (one workgroup per CU);
// otherwise the streaming tiled form.
hipError_t launch_wide_gemm(const WideArgs& a, int epi, hipStream_t s, int cus);
hipError_t launch_q8_quantize(const float* w, uint8_t* q, half_t* s, half_t* b, int N, int K, hipStream_t st);
hipError_t launch_q8_dequant(const uint8_t* q, const half_t* s, const half_t* b, half_t* w, int N, int K,
                             hipStream_t st);

}  // namespace esm
