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
// One workgroup per 32 cells of one pair row: the c channel rows of 64 bytes are read with
// coalesced 16-byte loads into LDS ([ch][cell], rows of 80 bytes); 8 threads per cell take the
// channels g + 8 e (consecutive rows for neighbouring threads: distinct banks), fp32 two-pass
// statistics over the 8 threads, and the normalised cell rows leave through LDS as whole
// 16-byte pieces.
constexpr int kCfCells = 32;
template <int CC>
__global__ __launch_bounds__(256) void ln_cf_to_cl_kernel(const half_t* __restrict__ x, int ldx,
                                                          const float* __restrict__ w, const float* __restrict__ b,
                                                          float eps, half_t* __restrict__ y, int B, int L) {
  constexpr int XS = kCfCells + 8;   // LDS row stride (halfs) of the channel-major tile
  constexpr int YS = CC + 8;         // LDS row stride (halfs) of the cell-major tile
  constexpr int PER = CC / 8;        // channels per thread
  __shared__ __align__(16) half_t xs[CC * XS];
  __shared__ __align__(16) half_t ys[kCfCells * YS];
  const int tid = threadIdx.x;
  const int tpl = (L + kCfCells - 1) / kCfCells;
  const long long ntiles = (long long)B * L * tpl;
  for (long long t = blockIdx.x; t < ntiles; t += gridDim.x) {
    const int bl = (int)(t / tpl);
    const int j0 = (int)(t - (long long)bl * tpl) * kCfCells;
    const int bi = bl / L, i = bl - bi * L;
    // 1. c rows x 32 cells (4 pieces of 8 cells per row)
    const rsrc_t rx = make_rsrc(x + ((size_t)bi * CC * L + i) * ldx + j0);
#pragma unroll
    for (int u = 0; u < CC * 4 / 256; u++) {
      const int q = tid + 256 * u, row = q >> 2, part = q & 3;
      const bool ok = j0 + 8 * part < ldx;
      st16(&xs[row * XS + 8 * part], bload16(rx, ok ? (uint32_t)((size_t)row * L * ldx + 8 * part) * 2u : kOOB));
    }
    __syncthreads();
    // 2. statistics and normalisation: thread (cell, g), channels g + 8 e
    const int cell = tid >> 3, gi = tid & 7;
    float v[PER];
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < PER; e++) {
      v[e] = (float)xs[(gi + 8 * e) * XS + cell];
      s += v[e];
    }
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    s += __shfl_xor(s, 4);
    const float mean = s * (1.0f / CC);
    float qv = 0.f;
#pragma unroll
    for (int e = 0; e < PER; e++) {
      v[e] -= mean;
      qv += v[e] * v[e];
    }
    qv += __shfl_xor(qv, 1);
    qv += __shfl_xor(qv, 2);
    qv += __shfl_xor(qv, 4);
    const float rstd = rsqrtf(qv * (1.0f / CC) + eps);
#pragma unroll
    for (int e = 0; e < PER; e++) {
      const int ch = gi + 8 * e;
      ys[cell * YS + ch] = (half_t)(v[e] * rstd * w[ch] + b[ch]);
    }
    __syncthreads();
    // 3. cell rows out: CC / 8 pieces of 16 bytes per cell
    half_t* yrow = y + ((size_t)bl * L + j0) * CC;
#pragma unroll
    for (int u = 0; u < kCfCells * (CC / 8) / 256; u++) {
      const int q = tid + 256 * u, c2 = q / (CC / 8), piece = q - c2 * (CC / 8);
      if (j0 + c2 < L) st16(yrow + (size_t)c2 * CC + 8 * piece, ld16(&ys[c2 * YS + 8 * piece]));
    }
    __syncthreads();  // xs and ys are rewritten by the next tile
  }
}

// ---- the wide GEMM ------------------------------------------------------------------------
namespace {
constexpr int WBM = 128;         // cells per tile
constexpr int WBN = 128;         // outputs per tile
constexpr int WBK = 32;          // k per stage
constexpr int WKS = WBK + 8;     // LDS row stride (halfs): 20 dwords
constexpr int WKC = WBK / 8;     // 16-byte chunks per row per stage
constexpr int WNT = 256;         // threads
constexpr int WOS = WBN + 8;     // LDS row stride (halfs) of the staged output tile
}  // namespace

template <int EPI, bool DUAL, bool A2SEP>
__global__ __launch_bounds__(WNT, 1) void wide_gemm_kernel(WideArgs p) {
  constexpr int NA = A2SEP ? 2 : 1;          // A panels per stage
  constexpr int NW = DUAL ? 2 : 1;           // W panels per stage
  constexpr int STAGE = (NA * WBM + NW * WBN) * WKS;
  constexpr int SMEM = (2 * STAGE > WBM * WOS) ? 2 * STAGE : WBM * WOS;
  constexpr int CH_A = WBM * WKC / WNT;      // 16-byte loads per thread per panel
  constexpr int CH_W = WBN * WKC / WNT;
  constexpr bool CM = EPI == kWideGateCM;    // channel-major output: D[cell][o]
  __shared__ __align__(16) half_t smem[SMEM];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int L = p.L, K = p.K;
  const int ntn = (p.N + WBN - 1) / WBN;
  const int t = xcd_remap(blockIdx.x, gridDim.x);
  const int mt = t / ntn, n0 = (t - mt * ntn) * WBN;
  const int bl = mt / p.tiles_per_line;      // (batch, line)
  const int pos0 = (mt - bl * p.tiles_per_line) * WBM;
  const int bi = bl / L, line = bl - bi * L;
  // cell of tile position m: (line, pos0 + m) in rows, or (pos0 + m, line) transposed
  const size_t cell0 = p.transpose ? ((size_t)bi * L + pos0) * L + line : ((size_t)bi * L + line) * L + pos0;
  const size_t cstride = p.transpose ? (size_t)L : 1;
  const int nvalid = L - pos0;               // cells of this tile inside the line

  const rsrc_t rA1 = make_rsrc(p.a1), rA2 = make_rsrc(A2SEP ? p.a2 : p.a1);
  const rsrc_t rW1 = make_rsrc(p.w1 + (size_t)n0 * K), rW2 = make_rsrc((DUAL ? p.w2 : p.w1) + (size_t)n0 * K);
  const int nk = (K + WBK - 1) / WBK;

  struct Regs {
    half8 a[NA][CH_A], w[NW][CH_W];
  };
  auto gload = [&](Regs& r, int kt) {
    const bool live = kt < nk;
#pragma unroll
    for (int u = 0; u < CH_A; u++) {
      const int id = tid + WNT * u, row = id / WKC, k = kt * WBK + (id % WKC) * 8;
      const bool ok = live && row < nvalid && k < K;
      const uint32_t off = ok ? (uint32_t)((cell0 + (size_t)row * cstride) * K + k) * 2u : kOOB;
      r.a[0][u] = bload16(rA1, off);
      if constexpr (A2SEP) r.a[1][u] = bload16(rA2, off);
    }
#pragma unroll
    for (int u = 0; u < CH_W; u++) {
      const int id = tid + WNT * u, row = id / WKC, k = kt * WBK + (id % WKC) * 8;
      const uint32_t off = live && n0 + row < p.N && k < K ? (uint32_t)(row * K + k) * 2u : kOOB;
      r.w[0][u] = bload16(rW1, off);
      if constexpr (DUAL) r.w[1][u] = bload16(rW2, off);
    }
  };
  auto swrite = [&](const Regs& r, int buf) {
    half_t* s = smem + buf * STAGE;
#pragma unroll
    for (int pa = 0; pa < NA; pa++)
#pragma unroll
      for (int u = 0; u < CH_A; u++) {
        const int id = tid + WNT * u;
        st16(s + (pa * WBM + id / WKC) * WKS + (id % WKC) * 8, r.a[pa][u]);
      }
#pragma unroll
    for (int pw = 0; pw < NW; pw++)
#pragma unroll
      for (int u = 0; u < CH_W; u++) {
        const int id = tid + WNT * u;
        st16(s + (NA * WBM + pw * WBN + id / WKC) * WKS + (id % WKC) * 8, r.w[pw][u]);
      }
  };

  f32x16 acc[2][2][2];  // [gemm][mi][ni]
#pragma unroll
  for (int g = 0; g < 2; g++)
#pragma unroll
    for (int mi = 0; mi < 2; mi++)
#pragma unroll
      for (int ni = 0; ni < 2; ni++)
#pragma unroll
        for (int e = 0; e < 16; e++) acc[g][mi][ni][e] = 0.f;

  auto compute = [&](int buf) {
    const half_t* s = smem + buf * STAGE;
#pragma unroll
    for (int kk = 0; kk < WBK / 16; kk++) {
      half8 af[NA][2], wf[NW][2];
#pragma unroll
      for (int pa = 0; pa < NA; pa++)
#pragma unroll
        for (int mi = 0; mi < 2; mi++)
          af[pa][mi] = ld16(s + (pa * WBM + wm * 64 + mi * 32 + (lane & 31)) * WKS + kk * 16 + 8 * (lane >> 5));
#pragma unroll
      for (int pw = 0; pw < NW; pw++)
#pragma unroll
        for (int ni = 0; ni < 2; ni++)
          wf[pw][ni] = ld16(s + (NA * WBM + pw * WBN + wn * 64 + ni * 32 + (lane & 31)) * WKS + kk * 16 + 8 * (lane >> 5));
#pragma unroll
      for (int g = 0; g < (DUAL ? 2 : 1); g++)
#pragma unroll
        for (int mi = 0; mi < 2; mi++)
#pragma unroll
          for (int ni = 0; ni < 2; ni++) {
            const half8 a = af[A2SEP ? g : 0][mi], w = wf[g][ni];
            acc[g][mi][ni] = CM ? mfma32(a, w, acc[g][mi][ni]) : mfma32(w, a, acc[g][mi][ni]);
          }
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

  // ---- epilogue: values in fp32, one rounding, staged in LDS ------------------------------
  // CM:  lane holds output o = lane % 32 (+ tile offsets) and 4 consecutive cells per group;
  //      staged as [o][cell].
  // else lane holds cell = lane % 32 and 4 consecutive outputs per group; staged [cell][o].
  half_t* os = smem;
#pragma unroll
  for (int mi = 0; mi < 2; mi++)
#pragma unroll
    for (int ni = 0; ni < 2; ni++)
#pragma unroll
      for (int g4 = 0; g4 < 4; g4++) {
        const int rq = acc_row32(4 * g4, lane);                      // first of 4 consecutive
        const int cl = CM ? wm * 64 + mi * 32 + rq : wm * 64 + mi * 32 + (lane & 31);
        const int ol = CM ? wn * 64 + ni * 32 + (lane & 31) : wn * 64 + ni * 32 + rq;
        half4 hv;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int c_e = CM ? cl + e : cl, o_e = CM ? ol : ol + e;  // this value's cell and output
          const float d1 = acc[0][mi][ni][4 * g4 + e];
          const float d2 = DUAL ? acc[1][mi][ni][4 * g4 + e] : 0.f;
          const bool cin = c_e < nvalid && n0 + o_e < p.N;
          const size_t cell = cell0 + (size_t)c_e * cstride;
          float v;
          if constexpr (EPI == kWideGateCM) {
            v = d1 * sigmoidf_fast(d2);
            if (p.mask) v *= cin ? (float)p.mask[cell] : 0.f;
          } else if constexpr (EPI == kWideResGate) {
            v = d1 * sigmoid_from_t(d2 * kNegLog2e);
            if (p.mask && p.out_mask) v *= cin ? (float)p.mask[cell] : 0.f;
            if (p.residual) v += cin ? (float)p.z[cell * p.ldo + n0 + o_e] : 0.f;
          } else if constexpr (EPI == kWideRelu) {
            v = fmaxf(d1, 0.f);
          } else if constexpr (EPI == kWideSwiglu) {
            v = d1 * sigmoidf_fast(d1) * d2;
          } else {  // kWideResid
            v = d1 + (cin ? (float)p.z[cell * p.ldo + n0 + o_e] : 0.f);
          }
          hv[e] = (half_t)v;
        }
        if (CM) {
          *reinterpret_cast<half4*>(os + ol * WOS + cl) = hv;  // [o][cell .. cell+3]
        } else {
          *reinterpret_cast<half4*>(os + cl * WOS + ol) = hv;  // [cell][o .. o+3]
        }
      }
  __syncthreads();
  if constexpr (CM) {
    // channel rows: output o -> plane a (o < c) or b, channel (n0 + o) % c; positions
    // pos0 .. pos0+127 of row `line`, up to ld (the padding columns get the zeros computed
    // for the cells past L).
#pragma unroll
    for (int u = 0; u < WBN * (WBM / 8) / WNT; u++) {
      const int id = tid + WNT * u, o = id / (WBM / 8), q = id - o * (WBM / 8);
      const int n = n0 + o;
      if (n >= p.N || pos0 + 8 * q >= p.ld) continue;
      half_t* plane = n < p.c ? p.plane_a : p.plane_b;
      const int ch = n < p.c ? n : n - p.c;
      st16(plane + (((size_t)bi * p.c + ch) * L + line) * p.ld + pos0 + 8 * q, ld16(os + o * WOS + 8 * q));
    }
  } else {
#pragma unroll
    for (int u = 0; u < WBM * (WBN / 8) / WNT; u++) {
      const int id = tid + WNT * u, c2 = id / (WBN / 8), q = id - c2 * (WBN / 8);
      if (c2 >= nvalid || n0 + 8 * q >= p.N) continue;
      st16(p.out + (cell0 + (size_t)c2 * cstride) * p.ldo + n0 + 8 * q, ld16(os + c2 * WOS + 8 * q));
    }
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
      hipLaunchKernelGGL((ln_rows_kernel<N, true>), dim3(grid), dim3(256), 0, s, x, x2, w, b, eps, out, rows); \
    else                                                                                                   \
      hipLaunchKernelGGL((ln_rows_kernel<N, false>), dim3(grid), dim3(256), 0, s, x, x2, w, b, eps, out, rows); \
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
      hipLaunchKernelGGL((ln_cf_to_cl_kernel<128>), dim3(grid), dim3(256), 0, s, x, ldx, w, b, eps, y, B, L);
      break;
    case 256:
      hipLaunchKernelGGL((ln_cf_to_cl_kernel<256>), dim3(grid), dim3(256), 0, s, x, ldx, w, b, eps, y, B, L);
      break;
    case 384:
      hipLaunchKernelGGL((ln_cf_to_cl_kernel<384>), dim3(grid), dim3(256), 0, s, x, ldx, w, b, eps, y, B, L);
      break;
    case 512:
      hipLaunchKernelGGL((ln_cf_to_cl_kernel<512>), dim3(grid), dim3(256), 0, s, x, ldx, w, b, eps, y, B, L);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

long long wide_gemm_blocks(const WideArgs& a) {
  return (long long)a.B * a.L * a.tiles_per_line * ((a.N + WBN - 1) / WBN);
}

hipError_t launch_wide_gemm(const WideArgs& a, int epi, hipStream_t s) {
  const dim3 grid((unsigned)wide_gemm_blocks(a)), block(WNT);
  const bool dual = a.w2 != nullptr, sep = a.a2 != nullptr && a.a2 != a.a1;
  switch (epi) {
    case kWideGateCM:
      if (!dual || sep) return hipErrorInvalidValue;
      hipLaunchKernelGGL((wide_gemm_kernel<kWideGateCM, true, false>), grid, block, 0, s, a);
      break;
    case kWideResGate:
      if (!dual || !sep) return hipErrorInvalidValue;
      hipLaunchKernelGGL((wide_gemm_kernel<kWideResGate, true, true>), grid, block, 0, s, a);
      break;
    case kWideRelu:
      if (dual) return hipErrorInvalidValue;
      hipLaunchKernelGGL((wide_gemm_kernel<kWideRelu, false, false>), grid, block, 0, s, a);
      break;
    case kWideSwiglu:
      if (!dual || sep) return hipErrorInvalidValue;
      hipLaunchKernelGGL((wide_gemm_kernel<kWideSwiglu, true, false>), grid, block, 0, s, a);
      break;
    case kWideResid:
      if (dual) return hipErrorInvalidValue;
      hipLaunchKernelGGL((wide_gemm_kernel<kWideResid, false, false>), grid, block, 0, s, a);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace esm
