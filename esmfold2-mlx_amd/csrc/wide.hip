// Wide path: the triangle update and the pair transition at pair widths other than the
// 128 channels the per-cell kernels (a), (c) and (e) are specialised for (ESMFold2's real
// trunk is 256 wide, mlx_trunk.py:3-5). The same arithmetic, split into generic pieces:
//
//   ln_rows        out[row] = fp16(LN(in[row]))  over C = 128 NCH channels (fp32 statistics)
//   ln_cf_to_cl    y[cell][ch] = fp16(LN over ch of x[ch][cell]): the contraction's
//                  channel-major output normalised and turned cell-major (the reference's
//                  ln_cf_to_cl, mlx_trunk_kernels.py:107-160)
//   wide_gemm      D = A1 . W1^T (and A2 . W2^T), fp16 operands, fp32 accumulation, with
//                  one fused epilogue:
//                    GATE_CM  a, b = A1 W_s^T * sigmoid(A1 W_g^T) * mask, stored channel-major
//                             (kernel (a)'s gate_cf, mlx_trunk_kernels.py:48-97)
//                    RESGATE  out = z + (y W_e^T) * sigmoid(n W_g^T) [* mask] (kernel (c)'s tail,
//                             mlx_trunk_kernels.py:224-227)
//                    RELU / SWIGLU   h = relu(A W1^T) or silu(A W1^T) * (A W2^T)
//                    RESID    out = z + A W^T (the transition's addmm residual, :239)
//
// wide_gemm tiles the cells as the per-cell kernels do: a tile is 128 consecutive cells of
// one line of the pair grid (a row; a column for the incoming direction's operands), times
// 128 outputs. Four waves in a 2 x 2 arrangement each own 64 cells x 64 outputs (2 x 2
// v_mfma_f32_32x32x16_f16 tiles per GEMM). K advances in stages of 32 through LDS (rows of
// 64 bytes, padded to 80: 16 consecutive rows start in 16 distinct 4-bank groups); stage
// kt+2 is requested into registers while stage kt is multiplied and stage kt+1 goes to the
// other LDS buffer. The result is staged in LDS and leaves as whole 16-byte pieces of rows
// (cell rows for the cell-major outputs, channel rows for GATE_CM). Tiles sharing A rows
// run on one XCD (their A panel is read once from HBM).
#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace esm {

// ---- LayerNorm over rows ------------------------------------------------------------------
// 16 lanes per row; lane l owns the 8-channel chunks l + 16 t (t < NCH). Input fp16, or the
// fp32 sum x + x2 (IN_F32). Two-pass fp32 statistics, one rounding to fp16.
template <int NCH, bool IN_F32>
__global__ __launch_bounds__(256) void ln_rows_kernel(const void* __restrict__ x, const float* __restrict__ x2,
                                                      const float* __restrict__ w, const float* __restrict__ b,
                                                      float eps, half_t* __restrict__ out, size_t rows) {
  constexpr int C = 128 * NCH;
  const int l16 = threadIdx.x & 15;
  float g[NCH][8], bb[NCH][8];
#pragma unroll
  for (int t = 0; t < NCH; t++)
#pragma unroll
    for (int e = 0; e < 8; e++) {
      g[t][e] = w[8 * (l16 + 16 * t) + e];
      bb[t][e] = b[8 * (l16 + 16 * t) + e];
    }
  for (size_t row = (size_t)blockIdx.x * 16 + (threadIdx.x >> 4); row < rows; row += (size_t)gridDim.x * 16) {
    float v[NCH][8];
#pragma unroll
    for (int t = 0; t < NCH; t++) {
      const size_t off = row * C + 8 * (l16 + 16 * t);
      if constexpr (IN_F32) {
        const float* xa = static_cast<const float*>(x) + off;
        const f32x4 a0 = *reinterpret_cast<const f32x4*>(xa), a1 = *reinterpret_cast<const f32x4*>(xa + 4);
        const f32x4 b0 = *reinterpret_cast<const f32x4*>(x2 + off), b1 = *reinterpret_cast<const f32x4*>(x2 + off + 4);
#pragma unroll
        for (int e = 0; e < 4; e++) {
          v[t][e] = a0[e] + b0[e];
          v[t][e + 4] = a1[e] + b1[e];
        }
      } else {
        const half8 h = ld16(static_cast<const half_t*>(x) + off);
#pragma unroll
        for (int e = 0; e < 8; e++) v[t][e] = (float)h[e];
      }
    }
    float s = 0.f;
#pragma unroll
    for (int t = 0; t < NCH; t++)
#pragma unroll
      for (int e = 0; e < 8; e++) s += v[t][e];
    const float mean = row16_sum(s) * (1.0f / C);
    float q = 0.f;
#pragma unroll
    for (int t = 0; t < NCH; t++)
#pragma unroll
      for (int e = 0; e < 8; e++) {
        v[t][e] -= mean;
        q += v[t][e] * v[t][e];
      }
    const float rstd = rsqrtf(row16_sum(q) * (1.0f / C) + eps);
#pragma unroll
    for (int t = 0; t < NCH; t++) {
      half8 o;
#pragma unroll
      for (int e = 0; e < 8; e++) o[e] = (half_t)(v[t][e] * rstd * g[t][e] + bb[t][e]);
      st16(out + row * C + 8 * (l16 + 16 * t), o);
    }
  }
}

// ---- LayerNorm over channels, channel-major -> cell-major -----------------------------------
// One 8-wave workgroup per 64 cells of one pair row. The c channel rows of 128 bytes arrive
// as coalesced 16-byte loads into LDS ([ch][cell], rows of 160 bytes: the 8 rows one pass of
// a transposing read touches cover the 64 banks once). Wave w takes the 16 cells
// 16 (w % 4) + n and the channel half w / 4; ds_read_b64_tr_b16 gives lane (g, n) =
// (lane / 16, lane % 16) the channels h c/2 + 4 g + 16 r .. +3 of its cell, so a lane holds
// c/8 channels of one cell after c/32 reads. Statistics from v_dot2_f32_f16 (sums of x and
// x^2) over the lane, the four lane groups (two exchanges) and the other channel half
// (through LDS), var = E[x^2] - E[x]^2. The normalised values go back to LDS cell-major as
// 8-byte pieces (4 channels) and leave as whole 16-byte pieces of the cell rows.
constexpr int kCfCells = 64;
constexpr int kCfThreads = 8 * kCfCells;  // two waves per 16 cells
template <int CC>
__global__ __launch_bounds__(kCfThreads) void ln_cf_to_cl_kernel(const half_t* __restrict__ x, int ldx,
                                                                 const float* __restrict__ w,
                                                                 const float* __restrict__ b, float eps,
                                                                 half_t* __restrict__ y, int B, int L) {
  constexpr int XS = kCfCells + 16;  // LDS row stride (halfs) of the channel-major tile
  constexpr int YS = CC + 8;         // LDS row stride (halfs) of the cell-major tile
  constexpr int NR = CC / 32;        // transposing reads per lane (4 channels each)
  constexpr int NCB = kCfCells / 16; // 16-cell blocks
  constexpr int NL = CC * (kCfCells / 8) / kCfThreads;  // 16-byte loads per thread
  static_assert(CC % 64 == 0 && NL >= 1, "whole reads and loads per thread");
  __shared__ __align__(16) half_t xs[CC * XS];
  __shared__ __align__(16) half_t ys[kCfCells * YS];
  __shared__ float st_s[2][kCfCells][2];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = tid >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int cb = wave % NCB, h = wave / NCB;
  const int cell = 16 * cb + n;
  const int ch0 = h * (CC / 2) + 4 * g;  // this lane's channels: ch0 + 16 r + e
  float gw[NR][4], gb[NR][4];
#pragma unroll
  for (int r = 0; r < NR; r++)
#pragma unroll
    for (int e = 0; e < 4; e++) {
      gw[r][e] = w[ch0 + 16 * r + e];
      gb[r][e] = b[ch0 + 16 * r + e];
    }
  const int tpl = (L + kCfCells - 1) / kCfCells;
  const long long ntiles = (long long)B * L * tpl;
  // XCD-aware order: a tile's 128-byte pieces of x are not line-aligned (rows of ld halfs),
  // so each line is shared with the neighbouring tile of the row or the next row; with
  // consecutive tiles on one XCD its L2 fetches the line once (dealt round-robin, the
  // reads were 1.8x the compulsory bytes)
  for (long long t = xcd_remap(blockIdx.x, gridDim.x); t < ntiles; t += gridDim.x) {
    const int bl = (int)(t / tpl);
    const int j0 = (int)(t - (long long)bl * tpl) * kCfCells;
    const int bi = bl / L, i = bl - bi * L;
    // 1. c rows x 64 cells (8 pieces of 8 cells per row). A wave's 64 lanes take 8 channel
    //    rows per load; the descriptor starts at the first of them, so every offset stays
    //    far below 2 GB whatever the size of the x planes.
    const half_t* xt = x + ((size_t)bi * CC * L + i) * ldx + j0;
    const int wu = __builtin_amdgcn_readfirstlane(tid >> 6);
#pragma unroll
    for (int u = 0; u < NL; u++) {
      const int q = tid + kCfThreads * u, row = q / (kCfCells / 8), part = q % (kCfCells / 8);
      const int row0 = (kCfThreads * u + 64 * wu) / (kCfCells / 8);  // the wave's first row
      const rsrc_t rx = make_rsrc(xt + (size_t)row0 * L * ldx);
      const bool ok = j0 + 8 * part < ldx;
      st16(&xs[row * XS + 8 * part],
           bload16(rx, ok ? (uint32_t)((size_t)(row - row0) * L * ldx + 8 * part) * 2u : kOOB));
    }
    __syncthreads();
    // 2. this lane's channels of its cell (the lane names the piece of 4 cells at channel
    //    ch0 + 16 r + n / 4, cells 16 cb + 4 (n % 4)); partial statistics, then the cell's
    half4 v[NR];
    float s = 0.f, q = 0.f;
#pragma unroll
    for (int r = 0; r < NR; r++) {
      v[r] = ds_read_tr16x4(&xs[(ch0 + 16 * r + (n >> 2)) * XS + 16 * cb + 4 * (n & 3)]);
      dot2_moments(v[r], s, q);
    }
    s += __shfl_xor(s, 16);
    q += __shfl_xor(q, 16);
    s += __shfl_xor(s, 32);
    q += __shfl_xor(q, 32);
    if (g == 0) {
      st_s[h][cell][0] = s;
      st_s[h][cell][1] = q;
    }
    __syncthreads();
    s += st_s[h ^ 1][cell][0];
    q += st_s[h ^ 1][cell][1];
    float rstd, shift;
    ln_scale_shift(s, q, 1.0f / CC, eps, rstd, shift);
    // 3. normalised pieces of 4 channels into the cell-major tile
#pragma unroll
    for (int r = 0; r < NR; r++) {
      half4 o;
#pragma unroll
      for (int e = 0; e < 4; e++) o[e] = ln_value(v[r][e], rstd, shift, gw[r][e], gb[r][e]);
      *reinterpret_cast<half4*>(&ys[cell * YS + ch0 + 16 * r]) = o;
    }
    __syncthreads();
    // 4. cell rows out: CC / 8 pieces of 16 bytes per cell
    half_t* yrow = y + ((size_t)bl * L + j0) * CC;
#pragma unroll
    for (int u = 0; u < kCfCells * (CC / 8) / kCfThreads; u++) {
      const int qq = tid + kCfThreads * u, c2 = qq / (CC / 8), piece = qq - c2 * (CC / 8);
      if (j0 + c2 < L) st16(yrow + (size_t)c2 * CC + 8 * piece, ld16(&ys[c2 * YS + 8 * piece]));
    }
    __syncthreads();  // xs, ys and the statistics are rewritten by the next tile
  }
}

// ---- the wide GEMM ------------------------------------------------------------------------
namespace {
constexpr int WBM = 128;         // cells per tile
constexpr int WNT = 512;         // threads: 8 waves, two per SIMD
}  // namespace

// The epilogue value of one output element from its fp32 sums d1 (GEMM 1) and d2 (GEMM 2),
// before the one rounding to fp16. `in` is false for the padding cells and outputs.
// zv is the residual z[cell][o] (RESGATE with residual, RESID; 0 for the padding).
template <int EPI>
DEV float wide_value(const WideArgs& p, float d1, float d2, size_t cell, bool in, float zv) {
  float v;
  if constexpr (EPI == kWideGateCM) {
    v = d1 * sigmoidf_fast(d2);
    if (p.mask) v *= in ? (float)p.mask[cell] : 0.f;
  } else if constexpr (EPI == kWideResGate) {
    v = d1 * sigmoid_from_t(d2 * kNegLog2e);
    if (p.mask && p.out_mask) v *= in ? (float)p.mask[cell] : 0.f;
    if (p.residual) v += zv;
  } else if constexpr (EPI == kWideRelu) {
    v = fmaxf(d1, 0.f);
  } else if constexpr (EPI == kWideSwiglu) {
    v = d1 * sigmoidf_fast(d1) * d2;
  } else {  // kWideResid
    v = d1 + zv;
  }
  return v;
}
template <int EPI>
constexpr bool wide_needs_z() { return EPI == kWideResGate || EPI == kWideResid; }


// Eight waves. DUAL (two GEMMs on the same outputs): a tile is 128 cells x 128 outputs;
// waves 0-3 compute GEMM 1 and waves 4-7 GEMM 2, each wave 64 cells x 64 outputs (2 x 2
// MFMA tiles, 64 accumulators), so both run at two waves per SIMD; the GEMM-2 waves hand
// their sums to the GEMM-1 waves through LDS (same wave-tile coordinates, so the same
// register index of the same lane: conflict-free 16-byte slots). Single GEMM: 128 cells x
// 256 outputs, 2 x 4 waves. Per stage of BK k: NA A panels of 128 cell rows and 256 weight
// rows (W1 then W2 for DUAL).
template <int EPI, bool DUAL, bool A2SEP, int BK>
__global__ __launch_bounds__(WNT, 1) void wide_gemm_kernel(WideArgs p) {
  constexpr int NA = A2SEP ? 2 : 1;            // A panels per stage
  constexpr int WNW = DUAL ? 2 : 4;            // waves along the outputs per GEMM
  constexpr int BN = 64 * WNW;                 // outputs per tile
  constexpr int WROWS = 256;                   // weight rows per stage
  constexpr int KS = BK + 8;                   // LDS row stride (halfs)
  constexpr int KC = BK / 8;                   // 16-byte chunks per row per stage
  constexpr int STAGE = (NA * WBM + WROWS) * KS;
  constexpr int OS = BN + 8;                   // output staging row stride (halfs)
  constexpr bool CM = EPI == kWideGateCM;      // channel-major output: D[cell][o]
  constexpr int OUT_HALFS = CM ? BN * (WBM + 8) : WBM * OS;
  constexpr int XCH_BYTES = DUAL ? 4 * 64 * 64 * 4 : 0;  // GEMM-2 sums of the 4 waves
  constexpr int SMEM_BYTES = 2 * STAGE * 2 > OUT_HALFS * 2 + XCH_BYTES ? 2 * STAGE * 2 : OUT_HALFS * 2 + XCH_BYTES;
  constexpr int CH_A = WBM * KC / WNT;         // 16-byte loads per thread per A panel
  constexpr int CH_W = WROWS * KC / WNT;
  static_assert(CH_A >= 1 && CH_W >= 1, "whole loads per thread");
  __shared__ __align__(16) char smem_c[SMEM_BYTES];
  half_t* smem = reinterpret_cast<half_t*>(smem_c);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int role = DUAL ? wave >> 2 : 0;                       // which GEMM this wave computes
  const int wm = DUAL ? (wave >> 1) & 1 : wave >> 2;           // 64-cell half of the tile
  const int wn = DUAL ? wave & 1 : wave & 3;                   // 64-output block
  const int L = p.L, K = p.K;
  const int ntn = (p.N + BN - 1) / BN;
  const int t = xcd_remap(blockIdx.x, gridDim.x);
  const int mt = t / ntn, n0 = (t - mt * ntn) * BN;
  const int bl = mt / p.tiles_per_line;      // (batch, line)
  const int pos0 = (mt - bl * p.tiles_per_line) * WBM;
  const int bi = bl / L, line = bl - bi * L;
  // cell of tile position m: (line, pos0 + m) in rows, or (pos0 + m, line) transposed
  const size_t cell0 = p.transpose ? ((size_t)bi * L + pos0) * L + line : ((size_t)bi * L + line) * L + pos0;
  const size_t cstride = p.transpose ? (size_t)L : 1;
  const int nvalid = L - pos0;               // cells of this tile inside the line

  // descriptors from the tile's first cell: offsets stay far below 2 GB at any grid size
  const rsrc_t rA1 = make_rsrc(p.a1 + cell0 * K), rA2 = make_rsrc((A2SEP ? p.a2 : p.a1) + cell0 * K);
  const rsrc_t rW1 = make_rsrc(p.w1 + (size_t)n0 * K), rW2 = make_rsrc((DUAL ? p.w2 : p.w1) + (size_t)n0 * K);
  const int nk = (K + BK - 1) / BK;

  struct Regs {
    half8 a[NA][CH_A], w[CH_W];
  };
  auto gload = [&](Regs& r, int kt) {
    const bool live = kt < nk;
#pragma unroll
    for (int u = 0; u < CH_A; u++) {
      const int id = tid + WNT * u, row = id / KC, k = kt * BK + (id % KC) * 8;
      const bool ok = live && row < nvalid && k < K;
      const uint32_t off = ok ? (uint32_t)((size_t)row * cstride * K + k) * 2u : kOOB;
      r.a[0][u] = bload16(rA1, off);
      if constexpr (A2SEP) r.a[1][u] = bload16(rA2, off);
    }
#pragma unroll
    for (int u = 0; u < CH_W; u++) {
      const int id = tid + WNT * u, row = id / KC, k = kt * BK + (id % KC) * 8;
      // DUAL: rows [0, 128) are W1's outputs n0.., rows [128, 256) W2's; else W1's n0 .. n0+255
      const int n = DUAL ? (row & (BN - 1)) : row;
      const bool ok = live && n0 + n < p.N && k < K;
      const uint32_t off = ok ? (uint32_t)(n * K + k) * 2u : kOOB;
      r.w[u] = bload16(DUAL && row >= BN ? rW2 : rW1, off);
    }
  };
  auto swrite = [&](const Regs& r, int buf) {
    half_t* s = smem + buf * STAGE;
#pragma unroll
    for (int pa = 0; pa < NA; pa++)
#pragma unroll
      for (int u = 0; u < CH_A; u++) {
        const int id = tid + WNT * u;
        st16(s + (pa * WBM + id / KC) * KS + (id % KC) * 8, r.a[pa][u]);
      }
#pragma unroll
    for (int u = 0; u < CH_W; u++) {
      const int id = tid + WNT * u;
      st16(s + (NA * WBM + id / KC) * KS + (id % KC) * 8, r.w[u]);
    }
  };

  f32x16 acc[2][2];  // [mi][ni]
#pragma unroll
  for (int mi = 0; mi < 2; mi++)
#pragma unroll
    for (int ni = 0; ni < 2; ni++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[mi][ni][e] = 0.f;

  const int arow0 = (A2SEP ? role * WBM : 0) + wm * 64;          // this wave's A rows in a stage
  const int wrow0 = NA * WBM + (DUAL ? role * BN : 0) + wn * 64;  // and its weight rows
  auto compute = [&](int buf) {
    const half_t* s = smem + buf * STAGE;
#pragma unroll
    for (int kk = 0; kk < BK / 16; kk++) {
      half8 af[2], wf[2];
#pragma unroll
      for (int mi = 0; mi < 2; mi++) af[mi] = ld16(s + (arow0 + mi * 32 + (lane & 31)) * KS + kk * 16 + 8 * (lane >> 5));
#pragma unroll
      for (int ni = 0; ni < 2; ni++) wf[ni] = ld16(s + (wrow0 + ni * 32 + (lane & 31)) * KS + kk * 16 + 8 * (lane >> 5));
#pragma unroll
      for (int mi = 0; mi < 2; mi++)
#pragma unroll
        for (int ni = 0; ni < 2; ni++)
          acc[mi][ni] = CM ? mfma32(af[mi], wf[ni], acc[mi][ni]) : mfma32(wf[ni], af[mi], acc[mi][ni]);
    }
  };

  Regs r0, r1;
  gload(r0, 0);
  gload(r1, 1);
  swrite(r0, 0);
  __syncthreads();
  for (int kt = 0; kt < nk; kt += 2) {
    gload(r0, kt + 2);
    compute(0);
    swrite(r1, 1);
    __syncthreads();
    gload(r1, kt + 3);
    compute(1);
    swrite(r0, 0);
    __syncthreads();
  }

  // ---- epilogue ---------------------------------------------------------------------------
  // DUAL: the GEMM-2 waves store their sums, the GEMM-1 waves read them at the same
  // (wave tile, register, lane) and compute every value; then all waves stage and store.
  f32x4* xch = reinterpret_cast<f32x4*>(smem_c + OUT_HALFS * 2);
  const int wt = wm * WNW + wn;  // wave-tile index within one GEMM
  if (DUAL && role == 1) {
#pragma unroll
    for (int mi = 0; mi < 2; mi++)
#pragma unroll
      for (int ni = 0; ni < 2; ni++)
#pragma unroll
        for (int g4 = 0; g4 < 4; g4++)
          xch[((wt * 4 + mi * 2 + ni) * 4 + g4) * 64 + lane] =
              f32x4{acc[mi][ni][4 * g4], acc[mi][ni][4 * g4 + 1], acc[mi][ni][4 * g4 + 2], acc[mi][ni][4 * g4 + 3]};
  }
  __syncthreads();
  // CM: lane holds output o = lane % 32 (+ tile offsets) and 4 consecutive cells per group;
  //     staged as [o][cell]. Else lane holds cell = lane % 32 and 4 consecutive outputs per
  //     group; staged as [cell][o].
  half4 hv[2][2][4];
  if (role == 0) {
#pragma unroll
    for (int mi = 0; mi < 2; mi++)
#pragma unroll
      for (int ni = 0; ni < 2; ni++)
#pragma unroll
        for (int g4 = 0; g4 < 4; g4++) {
          const int rq = acc_row32(4 * g4, lane);
          const int cl = CM ? wm * 64 + mi * 32 + rq : wm * 64 + mi * 32 + (lane & 31);
          const int ol = CM ? wn * 64 + ni * 32 + (lane & 31) : wn * 64 + ni * 32 + rq;
          f32x4 d2 = {0.f, 0.f, 0.f, 0.f};
          if (DUAL) d2 = xch[((wt * 4 + mi * 2 + ni) * 4 + g4) * 64 + lane];
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const int c_e = CM ? cl + e : cl, o_e = CM ? ol : ol + e;
            const bool in = c_e < nvalid && n0 + o_e < p.N;
            const size_t cell = cell0 + (size_t)c_e * cstride;
            const float zv = wide_needs_z<EPI>() && in && (EPI == kWideResid || p.residual)
                                 ? (float)p.z[cell * p.ldo + n0 + o_e] : 0.f;
            float v = wide_value<EPI>(p, acc[mi][ni][4 * g4 + e], d2[e], cell, in, zv);
            __asm__ volatile("" : "+v"(v));  // fp32 then fp16 at every position (as the weight-stationary form)
            hv[mi][ni][g4][e] = (half_t)v;
          }
        }
  }
  __syncthreads();  // the exchange area is free again
  half_t* os = smem;
  if (role == 0) {
#pragma unroll
    for (int mi = 0; mi < 2; mi++)
#pragma unroll
      for (int ni = 0; ni < 2; ni++)
#pragma unroll
        for (int g4 = 0; g4 < 4; g4++) {
          const int rq = acc_row32(4 * g4, lane);
          const int cl = CM ? wm * 64 + mi * 32 + rq : wm * 64 + mi * 32 + (lane & 31);
          const int ol = CM ? wn * 64 + ni * 32 + (lane & 31) : wn * 64 + ni * 32 + rq;
          if (CM)
            *reinterpret_cast<half4*>(os + ol * (WBM + 8) + cl) = hv[mi][ni][g4];  // [o][cell .. cell+3]
          else
            *reinterpret_cast<half4*>(os + cl * OS + ol) = hv[mi][ni][g4];         // [cell][o .. o+3]
        }
  }
  __syncthreads();
  if constexpr (CM) {
    // channel rows: output o -> plane a (o < c) or b, channel (n0 + o) % c; positions
    // pos0 .. pos0+127 of row `line`, up to ld (the padding columns get the zeros computed
    // for the cells past L).
#pragma unroll
    for (int u = 0; u < BN * (WBM / 8) / WNT; u++) {
      const int id = tid + WNT * u, o = id / (WBM / 8), q = id - o * (WBM / 8);
      const int n = n0 + o;
      if (n >= p.N || pos0 + 8 * q >= p.ld) continue;
      half_t* plane = n < p.c ? p.plane_a : p.plane_b;
      const int ch = n < p.c ? n : n - p.c;
      st16(plane + (((size_t)bi * p.c + ch) * L + line) * p.ld + pos0 + 8 * q, ld16(os + o * (WBM + 8) + 8 * q));
    }
  } else {
#pragma unroll
    for (int u = 0; u < WBM * (BN / 8) / WNT; u++) {
      const int id = tid + WNT * u, c2 = id / (BN / 8), q = id - c2 * (BN / 8);
      if (c2 >= nvalid || n0 + 8 * q >= p.N) continue;
      st16(p.out + (cell0 + (size_t)c2 * cstride) * p.ldo + n0 + 8 * q, ld16(os + c2 * OS + 8 * q));
    }
  }
}

// ---- the weight-stationary wide GEMM (K <= 256) --------------------------------------------
// Persistent: every workgroup owns a slice of the outputs (DUAL: 128 outputs of W1 and the
// same 128 of W2; single: 256 outputs of W1) and holds the slice's weight rows for the whole
// launch as v_mfma_f32_16x16x32_f16 fragments in registers: wave w takes 16 outputs of both
// GEMMs (DUAL) or 32 outputs (single), K / 4 registers either way. Tiles of 64 cells of one
// line stream through LDS with two tiles' loads in flight. A wave holds both GEMMs' sums for
// the same (cell, output) positions, so it finishes its outputs by itself: no exchange
// between waves, two barriers per tile, and one wave's epilogue runs under the other wave's
// MFMAs on the same SIMD. A tile is read by the S workgroups of the S slices, which are
// neighbours in the XCD-aware order (one L2 fetch).
namespace {
constexpr int SBM = 64;   // cells per tile
}  // namespace

// The epilogue of wide_value with the mask (HM) and the residual (RS) fixed per launch; mv is
// the cell's mask value (staged in LDS with the tile).
template <int EPI, bool HM, bool RS>
DEV float wide_value_u(float d1, float d2, float mv, bool in, float zv) {
  float v;
  if constexpr (EPI == kWideGateCM) {
    v = d1 * sigmoidf_fast(d2);
    if constexpr (HM) v *= in ? mv : 0.f;
  } else if constexpr (EPI == kWideResGate) {
    v = d1 * sigmoid_from_t(d2 * kNegLog2e);
    if constexpr (HM) v *= in ? mv : 0.f;
    if constexpr (RS) v += zv;
  } else if constexpr (EPI == kWideRelu) {
    v = fmaxf(d1, 0.f);
  } else if constexpr (EPI == kWideSwiglu) {
    v = d1 * sigmoidf_fast(d1) * d2;
  } else {  // kWideResid
    v = d1 + zv;
  }
  return v;
}

// FRAG (the channel-major epilogue only): tiles of 8 x 8 cells, operand rows line .. line+7
// by k pos0 .. pos0+7 (tile cell c = 8 dr + dc), and the a, b planes written in FragLayout,
// one whole 128-byte segment per channel and tile. HM (the gating epilogues only): the
// epilogue multiplies by the mask, whose values for a tile's cells are loaded with its A rows
// and staged in LDS; without it the kernel holds no mask code at all.
template <int EPI, bool DUAL, bool A2SEP, int KW, bool FRAG = false, bool HM = false>
__global__ __launch_bounds__(WNT, 1) void wide_gemm_ws_kernel(WideArgs p) {
  constexpr int K = 16 * KW;
  constexpr int KS = K / 32;                    // k-steps of the 16x16x32 MFMA
  constexpr int NA = A2SEP ? 2 : 1;
  constexpr int BN = DUAL ? 128 : 256;          // outputs per slice
  constexpr int NOB = DUAL ? 1 : 2;             // 16-output blocks per wave
  constexpr int AS = K + 8;                     // LDS row stride (halfs) of an A tile
  constexpr int A_HALFS = NA * SBM * AS;
  constexpr bool CM = EPI == kWideGateCM;
  constexpr bool ZR = wide_needs_z<EPI>();      // the residual comes in with the A tile
  constexpr int OS = CM ? SBM + 8 : BN + 8;     // staging row stride: [o][cell] or [cell][o]
  constexpr int OUT_HALFS = CM ? BN * OS : SBM * OS;
  constexpr int WST_HALFS = 64 * AS;            // start-up: 64 weight rows at a time
  constexpr int MAIN_BYTES = A_HALFS * 2 + OUT_HALFS * 2;
  constexpr int SMEM_BYTES = MAIN_BYTES > WST_HALFS * 2 ? MAIN_BYTES : WST_HALFS * 2;
  constexpr int CH_A = SBM * (K / 8) / WNT;     // 16-byte loads per thread per A tile
  static_assert(CH_A >= 1 && SBM * (K / 8) % WNT == 0, "whole loads per thread");
  static_assert(KS >= 1 && K % 32 == 0, "K a multiple of 32");
  static_assert(!(CM && ZR), "no residual with channel-major planes");
  static_assert(!FRAG || CM, "the fragment layout is for the channel-major planes");
  __shared__ __align__(16) char smem_c[SMEM_BYTES];
  __shared__ __align__(16) float m_s[HM ? SBM : 4];  // the tile's mask values
  half_t* a_s = reinterpret_cast<half_t*>(smem_c);
  half_t* os = reinterpret_cast<half_t*>(smem_c + A_HALFS * 2);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, q4 = lane >> 4;
  const int L = p.L;
  const int S = (p.N + BN - 1) / BN;            // slices
  const int lg = xcd_remap(blockIdx.x, gridDim.x);
  const int slice = lg % S;
  const int n0 = slice * BN;
  const int stride = gridDim.x / S;             // tile groups
  const int tpl = FRAG ? (L + 7) / 8 : (L + SBM - 1) / SBM;  // FRAG: tiles per dimension
  const int ntiles = FRAG ? p.B * tpl * tpl : p.B * L * tpl;
  // first output (in the slice) of 16-output block b of this wave
  const int ob0 = DUAL ? 16 * wave : 32 * wave;

  // fragment set f: DUAL: W1 (f = 0), W2 (f = 1) for outputs ob0 .. ob0+15;
  // single: W1 for outputs ob0 + 16 f .. +15. Lane: row l16 of the set, k = 32 ks + 8 q4 + e.
  half8 wf[2][KS];

  auto tile_coords = [&](int tile_v, int& bi, int& line, int& pos0) {
    const int tile = __builtin_amdgcn_readfirstlane(tile_v);  // uniform: keep the division scalar
    if constexpr (FRAG) {
      bi = tile / (tpl * tpl);
      const int t = tile - bi * tpl * tpl, tr = t / tpl;
      line = 8 * tr;
      pos0 = 8 * (t - tr * tpl);
    } else {
      const int bl = tile / tpl;
      pos0 = (tile - bl * tpl) * SBM;
      bi = bl / L;
      line = bl - bi * L;
    }
  };
  auto cell_of = [&](int bi, int line, int pos) -> size_t {
    return p.transpose ? ((size_t)bi * L + pos) * L + line : ((size_t)bi * L + line) * L + pos;
  };
  // tile cell c: its (line, position) and whether it lies inside the grid
  auto tcell = [&](int line, int pos0, int c, int& ln, int& ps) -> bool {
    if constexpr (FRAG) {
      ln = line + (c >> 3);
      ps = pos0 + (c & 7);
      return ln < L && ps < L;
    } else {
      ln = line;
      ps = pos0 + c;
      return ps < L;
    }
  };
  static_assert(!HM || EPI == kWideGateCM || EPI == kWideResGate, "the mask is a gating epilogue's");
  struct Regs {
    half8 a[NA][CH_A];
    half4 z[ZR ? NOB : 1][ZR ? 4 : 1];          // z[cell 16 cb + l16][outputs ob + 4 q4 .. +3]
    uint16_t mk;                                // threads 0 .. SBM-1: the mask of tile cell tid
  };
  // One tile's loads: the A rows (row-contiguous 16-byte pieces), and the residual pieces
  // this lane adds, 8 bytes each. The descriptors start at the tile's first cell (line, pos0):
  // every other cell of the tile lies after it (at most a few lines further), so the
  // offsets stay far below 2 GB at any grid size.
  auto gload = [&](Regs& r, int tile) {
    const bool live = tile < ntiles;
    int bi, line, pos0;
    tile_coords(live ? tile : 0, bi, line, pos0);
    const size_t c0 = cell_of(bi, line, pos0);
    const rsrc_t rA1 = make_rsrc(p.a1 + c0 * K), rA2 = make_rsrc((A2SEP ? p.a2 : p.a1) + c0 * K);
#pragma unroll
    for (int u = 0; u < CH_A; u++) {
      const int id = tid + WNT * u, row = id / (K / 8), j = id - row * (K / 8);
      int ln, ps;
      const bool ok = tcell(line, pos0, row, ln, ps) && live;
      const uint32_t off = ok ? (uint32_t)((cell_of(bi, ln, ps) - c0) * K + 8 * j) * 2u : kOOB;
      r.a[0][u] = bload16(rA1, off);
      if constexpr (A2SEP) r.a[1][u] = bload16(rA2, off);
    }
    if constexpr (HM) {  // one mask value per tile cell, loaded with the A rows
      const rsrc_t rM = make_rsrc(p.mask + c0);
      int ln, ps;
      const bool ok = live && tid < SBM && tcell(line, pos0, tid, ln, ps);
      r.mk = bload2(rM, ok ? (uint32_t)(cell_of(bi, ln, ps) - c0) * 2u : kOOB);
    }
    if constexpr (ZR) {
      const bool want = EPI == kWideResid || p.residual;
      const rsrc_t rZ = make_rsrc(p.z + c0 * p.ldo);
#pragma unroll
      for (int b = 0; b < NOB; b++)
#pragma unroll
        for (int cb = 0; cb < 4; cb++) {
          const int c = 16 * cb + l16, o = n0 + ob0 + 16 * b + 4 * q4;
          const bool ok = want && live && pos0 + c < L && o < p.N;
          const uint32_t off = ok ? (uint32_t)((cell_of(bi, line, pos0 + c) - c0) * p.ldo + o) * 2u : kOOB;
          r.z[b][cb] = __builtin_bit_cast(half4, __builtin_amdgcn_raw_buffer_load_b64(rZ, (int)off, 0, 0));
        }
    }
  };

  // one tile: A tiles to LDS, the MFMAs, each wave's own epilogue into the staging tile, stores
  auto run_tile = [&](int tile, const Regs& ra) {
    int bi, line, pos0;
    tile_coords(tile, bi, line, pos0);
    const int nvalid = L - pos0;
#pragma unroll
    for (int pa = 0; pa < NA; pa++)
#pragma unroll
      for (int u = 0; u < CH_A; u++) {
        const int id = tid + WNT * u, row = id / (K / 8), j = id - row * (K / 8);
        st16(a_s + (pa * SBM + row) * AS + 8 * j, ra.a[pa][u]);
      }
    if constexpr (HM)
      if (tid < SBM) m_s[tid] = h2f(ra.mk);
    __syncthreads();  // the A tiles are in LDS; the previous tile's staging reads are done
    f32x4 acc[2][4];
#pragma unroll
    for (int f = 0; f < 2; f++)
#pragma unroll
      for (int cb = 0; cb < 4; cb++) acc[f][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ks++)
#pragma unroll
      for (int cb = 0; cb < 4; cb++) {
        const half8 a1 = ld16(a_s + (16 * cb + l16) * AS + 32 * ks + 8 * q4);
        const half8 a2 = A2SEP ? ld16(a_s + (SBM + 16 * cb + l16) * AS + 32 * ks + 8 * q4) : a1;
#pragma unroll
        for (int f = 0; f < 2; f++) {
          const half8 af = (A2SEP && f == 1) ? a2 : a1;
          // CM: D[cell][output] (a lane ends with 4 consecutive cells of one output);
          // otherwise D[output][cell] (4 consecutive outputs of one cell)
          acc[f][cb] = CM ? mfma16(af, wf[f][ks], acc[f][cb]) : mfma16(wf[f][ks], af, acc[f][cb]);
        }
      }
    // the MFMA block is scheduled on its own (LDS reads kept ahead of their products), apart
    // from the epilogue's transcendental arithmetic
    __builtin_amdgcn_sched_barrier(0);
    auto finish = [&](auto rs) {
      constexpr bool RS = decltype(rs)::value;
      f32x4 mv[4];  // the mask of this lane's cells (all four LDS reads issued before the first use)
#pragma unroll
      for (int cb = 0; cb < 4; cb++) {
        if constexpr (!HM)
          mv[cb] = f32x4{1.f, 1.f, 1.f, 1.f};
        else if constexpr (CM)
          mv[cb] = *reinterpret_cast<const f32x4*>(m_s + 16 * cb + 4 * q4);
        else
          mv[cb] = f32x4{m_s[16 * cb + l16], m_s[16 * cb + l16], m_s[16 * cb + l16], m_s[16 * cb + l16]};
      }
#pragma unroll
      for (int b = 0; b < NOB; b++)
#pragma unroll
        for (int cb = 0; cb < 4; cb++) {
          half4 hv;
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const int cl = CM ? 16 * cb + 4 * q4 + e : 16 * cb + l16;
            const int ol = CM ? ob0 + l16 : ob0 + 16 * b + 4 * q4 + e;
            int ln, ps;
            const bool in = (FRAG ? tcell(line, pos0, cl, ln, ps) : cl < nvalid) && n0 + ol < p.N;
            if constexpr (!FRAG) {
              ln = line;
              ps = pos0 + cl;
            }
            const float d1 = acc[DUAL ? 0 : b][cb][e], d2 = DUAL ? acc[1][cb][e] : 0.f;
            const float zv = ZR ? (float)ra.z[ZR ? b : 0][ZR ? cb : 0][e] : 0.f;  // zeros past the ends
            float v = wide_value_u<EPI, HM, RS>(d1, d2, mv[cb][e], in, zv);
            // fp32 first, then fp16, at every position: left to itself the compiler fuses the
            // last multiply with the conversion (one rounding) at some accumulator positions
            // only, so a cell's bits would depend on where the tiling puts it
            __asm__ volatile("" : "+v"(v));
            hv[e] = (half_t)v;
          }
          if (CM)
            *reinterpret_cast<half4*>(os + (ob0 + l16) * OS + 16 * cb + 4 * q4) = hv;
          else
            *reinterpret_cast<half4*>(os + (16 * cb + l16) * OS + ob0 + 16 * b + 4 * q4) = hv;
        }
    };
    if (EPI == kWideResid || (EPI == kWideResGate && p.residual))
      finish(std::true_type{});
    else
      finish(std::false_type{});
    __syncthreads();  // the staged tile is complete; every wave is done with the A tiles
    if constexpr (CM && FRAG) {
      // chunk q of a channel's staged row: operand row line + q, k pos0 .. pos0+7, lane
      // (line + q) % 32 + 32 (pos0 / 8 % 2) of tile ((line + q) / 32, pos0 / 16)
      const size_t plane_h = (size_t)p.rbn * p.kbn * FragLayout::kTileHalfs;
      const size_t tile_h = ((size_t)(line >> 5) * p.kbn + (pos0 >> 4)) * FragLayout::kTileHalfs +
                            (size_t)((line & 31) + 32 * ((pos0 >> 3) & 1)) * 8;
      for (int id = tid; id < BN * (SBM / 8); id += WNT) {
        const int o = id / (SBM / 8), q = id - o * (SBM / 8);
        const int n = n0 + o;
        if (n >= p.N) continue;
        half_t* plane = n < p.c ? p.plane_a : p.plane_b;
        const int ch = n < p.c ? n : n - p.c;
        st16(plane + ((size_t)bi * p.c + ch) * plane_h + tile_h + 8 * q, ld16(os + o * OS + 8 * q));
      }
    } else if constexpr (CM) {
      for (int id = tid; id < BN * (SBM / 8); id += WNT) {
        const int o = id / (SBM / 8), q = id - o * (SBM / 8);
        const int n = n0 + o;
        if (n >= p.N || pos0 + 8 * q >= p.ld) continue;
        half_t* plane = n < p.c ? p.plane_a : p.plane_b;
        const int ch = n < p.c ? n : n - p.c;
        st16(plane + (((size_t)bi * p.c + ch) * L + line) * p.ld + pos0 + 8 * q, ld16(os + o * OS + 8 * q));
      }
    } else {
      for (int id = tid; id < SBM * (BN / 8); id += WNT) {
        const int c2 = id / (BN / 8), q = id - c2 * (BN / 8);
        if (c2 >= nvalid || n0 + 8 * q >= p.N) continue;
        st16(p.out + cell_of(bi, line, pos0 + c2) * p.ldo + n0 + 8 * q, ld16(os + c2 * OS + 8 * q));
      }
    }
  };

  // Weights: the slice's rows (DUAL: W1's BN, then W2's BN) are requested at once, the first
  // tile's loads behind them, then staged through LDS 64 rows at a time so that the global
  // reads stay row-contiguous (fragment-pattern reads straight from global memory were no
  // faster: the start-up is bound by the 128 KB each workgroup pulls through its L1).
  constexpr int WROWS = DUAL ? 2 * BN : BN;
  constexpr int WCH = 64 * (K / 8) / WNT;       // 16-byte chunks per thread per 64 rows
  static_assert(WCH >= 1 && 64 * (K / 8) % WNT == 0, "whole weight chunks per thread");
  const int tg = lg / S;
  Regs r0, r1;
  {
    const rsrc_t rW1 = make_rsrc(p.w1), rW2 = make_rsrc(DUAL ? p.w2 : p.w1);
    half8 wst[WROWS / 64][WCH];
#pragma unroll
    for (int r = 0; r < WROWS / 64; r++)
#pragma unroll
      for (int q = 0; q < WCH; q++) {
        const int id = tid + WNT * q, rr = id / (K / 8), j = id - rr * (K / 8);
        const int g = DUAL ? r * 64 / BN : 0;                // W1 or W2 (64 divides BN; unrolled r)
        const int n = r * 64 - g * BN + rr;                  // row of that matrix in the slice
        const uint32_t off = n0 + n < p.N ? (uint32_t)(((size_t)(n0 + n) * K + 8 * j) * 2) : kOOB;
        wst[r][q] = bload16(g ? rW2 : rW1, off);
      }
    gload(r0, tg);
#pragma unroll
    for (int r = 0; r < WROWS / 64; r++) {
#pragma unroll
      for (int q = 0; q < WCH; q++) {
        const int id = tid + WNT * q, rr = id / (K / 8), j = id - rr * (K / 8);
        st16(a_s + rr * AS + 8 * j, wst[r][q]);
      }
      __syncthreads();
#pragma unroll
      for (int f = 0; f < 2; f++) {
        const int sb = DUAL ? f * BN + ob0 : ob0 + 16 * f;  // the set's first slice row
        if (sb >= r * 64 && sb < r * 64 + 64) {
#pragma unroll
          for (int ks = 0; ks < KS; ks++) wf[f][ks] = ld16(a_s + (sb - r * 64 + l16) * AS + 32 * ks + 8 * q4);
        }
      }
      __syncthreads();
    }
  }
  gload(r1, tg + stride);

  // Two tiles' loads in flight: a tile's registers are reloaded (two tiles ahead) only after
  // its epilogue has used them; the next tile's loads were issued before this tile's stores,
  // so waiting for them never waits for the stores. The A tiles are rewritten only after the
  // second barrier of the previous tile (every wave's MFMAs done), and the staging tile only
  // after the first barrier of the next tile (every thread's stores read).
  for (int tile = tg; tile < ntiles; tile += 2 * stride) {
    run_tile(tile, r0);
    gload(r0, tile + 2 * stride);
    if (tile + stride < ntiles) run_tile(tile + stride, r1);
    gload(r1, tile + 3 * stride);
  }
}

// ---- launchers ----------------------------------------------------------------------------
hipError_t launch_ln_rows(const void* x, const float* x2, bool in_f32, const float* w, const float* b, float eps,
                          half_t* out, size_t rows, int C, hipStream_t s) {
  const size_t blocks = (rows + 15) / 16;
  const int grid = (int)(blocks < 4096 ? blocks : 4096);
#define LN_ROWS_CASE(N)                                                                                    \
  case N:                                                                                                  \
    if (in_f32)                                                                                            \
      ESM_LAUNCH((ln_rows_kernel<N, true>), dim3(grid), dim3(256), 0, s, x, x2, w, b, eps, out, rows); \
    else                                                                                                   \
      ESM_LAUNCH((ln_rows_kernel<N, false>), dim3(grid), dim3(256), 0, s, x, x2, w, b, eps, out, rows); \
    break;
  switch (C / 128) {
    LN_ROWS_CASE(1)
    LN_ROWS_CASE(2)
    LN_ROWS_CASE(3)
    LN_ROWS_CASE(4)
    default:
      return hipErrorInvalidValue;
  }
#undef LN_ROWS_CASE
  return hipGetLastError();
}

hipError_t launch_ln_cf_to_cl(const half_t* x, int ldx, const float* w, const float* b, float eps, half_t* y, int B,
                              int L, int c, hipStream_t s) {
  const long long tiles = (long long)B * L * ((L + kCfCells - 1) / kCfCells);
  const int grid = (int)(tiles < 16384 ? tiles : 16384);
  switch (c) {
    case 128:
      ESM_LAUNCH((ln_cf_to_cl_kernel<128>), dim3(grid), dim3(kCfThreads), 0, s, x, ldx, w, b, eps, y, B, L);
      break;
    case 256:
      ESM_LAUNCH((ln_cf_to_cl_kernel<256>), dim3(grid), dim3(kCfThreads), 0, s, x, ldx, w, b, eps, y, B, L);
      break;
    case 384:
      ESM_LAUNCH((ln_cf_to_cl_kernel<384>), dim3(grid), dim3(kCfThreads), 0, s, x, ldx, w, b, eps, y, B, L);
      break;
    case 512:
      ESM_LAUNCH((ln_cf_to_cl_kernel<512>), dim3(grid), dim3(kCfThreads), 0, s, x, ldx, w, b, eps, y, B, L);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

long long wide_gemm_blocks(const WideArgs& a) {
  const int bn = a.w2 != nullptr ? 128 : 256;
  return (long long)a.B * a.L * a.tiles_per_line * ((a.N + bn - 1) / bn);
}

constexpr int kWideBK = 64;

// The weight-stationary form for K = 128 or 256: a persistent grid of whole slice groups.
static hipError_t launch_wide_gemm_ws(const WideArgs& a, int epi, int cus, hipStream_t s) {
  const bool dual = a.w2 != nullptr, sep = a.a2 != nullptr && a.a2 != a.a1;
  const int bn = dual ? 128 : 256;
  const int S = (a.N + bn - 1) / bn;
  const long long tpd = (a.L + 7) / 8;
  const long long tiles = a.frag ? a.B * tpd * tpd : (long long)a.B * a.L * ((a.L + SBM - 1) / SBM);
  long long groups = (cus > S ? cus : S) / S;   // one workgroup per CU
  groups -= groups % kNumXcd == 0 || groups < kNumXcd ? 0 : groups % kNumXcd;
  if (groups > tiles) groups = tiles;
  const dim3 grid((unsigned)(groups * S)), block(WNT);
#define WS_CASES(KW)                                                                                          \
  switch (epi) {                                                                                             \
    case kWideGateCM:                                                                                        \
      if (!dual || sep) return hipErrorInvalidValue;                                                         \
      if (a.frag && a.mask)                                                                                  \
        ESM_LAUNCH((wide_gemm_ws_kernel<kWideGateCM, true, false, KW, true, true>), grid, block, 0, s, a);   \
      else if (a.frag)                                                                                       \
        ESM_LAUNCH((wide_gemm_ws_kernel<kWideGateCM, true, false, KW, true>), grid, block, 0, s, a);         \
      else if (a.mask)                                                                                       \
        ESM_LAUNCH((wide_gemm_ws_kernel<kWideGateCM, true, false, KW, false, true>), grid, block, 0, s, a);  \
      else                                                                                                   \
        ESM_LAUNCH((wide_gemm_ws_kernel<kWideGateCM, true, false, KW>), grid, block, 0, s, a);               \
      break;                                                                                                 \
    case kWideResGate:                                                                                       \
      if (!dual || !sep) return hipErrorInvalidValue;                                                        \
      if (a.mask && a.out_mask)                                                                              \
        ESM_LAUNCH((wide_gemm_ws_kernel<kWideResGate, true, true, KW, false, true>), grid, block, 0, s, a);  \
      else                                                                                                   \
        ESM_LAUNCH((wide_gemm_ws_kernel<kWideResGate, true, true, KW>), grid, block, 0, s, a);               \
      break;                                                                                                 \
    case kWideRelu:                                                                                          \
      if (dual) return hipErrorInvalidValue;                                                                 \
      ESM_LAUNCH((wide_gemm_ws_kernel<kWideRelu, false, false, KW>), grid, block, 0, s, a);          \
      break;                                                                                                 \
    case kWideSwiglu:                                                                                        \
      if (!dual || sep) return hipErrorInvalidValue;                                                         \
      ESM_LAUNCH((wide_gemm_ws_kernel<kWideSwiglu, true, false, KW>), grid, block, 0, s, a);         \
      break;                                                                                                 \
    case kWideResid:                                                                                         \
      if (dual) return hipErrorInvalidValue;                                                                 \
      ESM_LAUNCH((wide_gemm_ws_kernel<kWideResid, false, false, KW>), grid, block, 0, s, a);         \
      break;                                                                                                 \
    default:                                                                                                 \
      return hipErrorInvalidValue;                                                                           \
  }
  if (a.K == 128) {
    WS_CASES(8)
  } else {
    WS_CASES(16)
  }
#undef WS_CASES
  return hipGetLastError();
}

hipError_t launch_wide_gemm(const WideArgs& a, int epi, hipStream_t s, int cus) {
  if ((a.K == 128 || a.K == 256) && cus > 0) return launch_wide_gemm_ws(a, epi, cus, s);
  if (a.frag) return hipErrorInvalidValue;  // the fragment layout is written by the weight-stationary form only
  const dim3 grid((unsigned)wide_gemm_blocks(a)), block(WNT);
  const bool dual = a.w2 != nullptr, sep = a.a2 != nullptr && a.a2 != a.a1;
  switch (epi) {
    case kWideGateCM:
      if (!dual || sep) return hipErrorInvalidValue;
      ESM_LAUNCH((wide_gemm_kernel<kWideGateCM, true, false, kWideBK>), grid, block, 0, s, a);
      break;
    case kWideResGate:
      if (!dual || !sep) return hipErrorInvalidValue;
      ESM_LAUNCH((wide_gemm_kernel<kWideResGate, true, true, kWideBK>), grid, block, 0, s, a);
      break;
    case kWideRelu:
      if (dual) return hipErrorInvalidValue;
      ESM_LAUNCH((wide_gemm_kernel<kWideRelu, false, false, kWideBK>), grid, block, 0, s, a);
      break;
    case kWideSwiglu:
      if (!dual || sep) return hipErrorInvalidValue;
      ESM_LAUNCH((wide_gemm_kernel<kWideSwiglu, true, false, kWideBK>), grid, block, 0, s, a);
      break;
    case kWideResid:
      if (dual) return hipErrorInvalidValue;
      ESM_LAUNCH((wide_gemm_kernel<kWideResid, false, false, kWideBK>), grid, block, 0, s, a);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace esm
