// Kernel (c): norm_mix LayerNorm over the c channels of the channel-major
// contraction output -> proj_emit (MFMA) -> * sigmoid(proj_gate(LN_in(z))) (MFMA)
// [-> * mask] [-> + z], written cell-major.
//
// Persistent like kernel (a): proj_emit and proj_gate weights stay in VGPRs; a
// tile is 64 cells of one row i of the pair grid, cells (i, pos0..pos0+63).
// Per tile:
//   1. x[:, i, pos0:pos0+64] arrives as 128 channel rows of 128 contiguous bytes
//      (16-byte loads) and is transposed into an LDS tile [cell][c];
//   2. z's 64 cells are read (256 contiguous bytes each), LayerNormed (norm_start)
//      into a second LDS tile; the raw z stays in registers for the residual;
//   3. norm_mix is applied in place to the x tile (fp32 statistics);
//   4. two MFMA GEMMs (emit on LN(x), gate on LN(z)), gate applied in fp32 from
//      the accumulators, the fp32 update staged in LDS;
//   5. the update (+ z) is rounded once to fp16 and stored as 256-byte cell rows.
// The output gate is recomputed from z rather than stored by kernel (a): z is
// 2C bytes per cell, a stored gate would cost a write plus a read of 2C bytes.
#include "common.h"
#include "kernels.h"

namespace esm {

namespace {
constexpr int C = 128;          // pair channels (output)
constexpr int CL = 128;         // latent channels (contraction output)
constexpr int TM = kCellTile;   // cells per tile
constexpr int XS = CL + 8;      // LDS row stride (halfs), x tile
constexpr int NS = C + 8;       // LDS row stride (halfs), LN(z) tile
constexpr int OS = C + 4;       // LDS row stride (floats), update staging
}  // namespace

__global__ __launch_bounds__(256, 2) void tmu_epilogue_kernel(EpilogueArgs p) {
  __shared__ __align__(16) half_t x_s[TM * XS];
  __shared__ __align__(16) half_t n_s[TM * NS];
  __shared__ __align__(16) float o_s[TM * OS];
  __shared__ float m_s[TM];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int L = p.L;

  // Weights as MFMA A-fragments: output channels o in [32 wave, 32 wave + 32).
  half8 we[CL / 16], wg[C / 16];
  {
    const int o = 32 * wave + (lane & 31);
#pragma unroll
    for (int ks = 0; ks < CL / 16; ks++) we[ks] = ld16(p.w_emit + (size_t)o * CL + ks * 16 + 8 * (lane >> 5));
#pragma unroll
    for (int ks = 0; ks < C / 16; ks++) wg[ks] = ld16(p.w_gate + (size_t)o * C + ks * 16 + 8 * (lane >> 5));
  }
  const int ch0 = (lane & 15) * 8;
  float gin[8], bin[8], gmx[8], bmx[8];
#pragma unroll
  for (int e = 0; e < 8; e++) {
    gin[e] = p.ln_in_w[ch0 + e];
    bin[e] = p.ln_in_b[ch0 + e];
    gmx[e] = p.ln_mix_w[ch0 + e];
    bmx[e] = p.ln_mix_b[ch0 + e];
  }

  for (int tile = blockIdx.x; tile < p.ntiles; tile += gridDim.x) {
    const int bl = tile / p.tiles_per_line;
    const int pos0 = (tile - bl * p.tiles_per_line) * TM;
    const int bi = bl / L, i = bl - bi * L;
    const size_t row_cells = ((size_t)bi * L + i) * L;  // index of cell (i, 0)

    // 1. x rows -> LDS [cell][d]
#pragma unroll
    for (int u = 0; u < (CL * TM / 8) / 256; u++) {
      const int id = tid + 256 * u;
      const int d = id >> 3, q = id & 7;
      const int pos = pos0 + q * 8;
      half8 v = zero_half8();
      if (pos < L) v = ld16(p.x + (((size_t)bi * CL + d) * L + i) * p.ldx + pos);
#pragma unroll
      for (int e = 0; e < 8; e++) x_s[(q * 8 + e) * XS + d] = v[e];
    }
    // 2. z -> LN_in -> LDS; raw z kept for the residual
    half8 zr[4];
#pragma unroll
    for (int it = 0; it < 4; it++) {
      const int cl = (tid >> 4) + 16 * it;
      const int pos = pos0 + cl;
      zr[it] = zero_half8();
      float mval = 1.f;
      if (pos < L) {
        zr[it] = ld16(p.z + (row_cells + pos) * C + ch0);
        if (p.mask) mval = (float)p.mask[row_cells + pos];
      }
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; e++) v[e] = (float)zr[it][e];
      ln_row128(v, gin, bin, p.eps_in);
      half8 o;
#pragma unroll
      for (int e = 0; e < 8; e++) o[e] = (half_t)v[e];
      st16(&n_s[cl * NS + ch0], o);
      if ((lane & 15) == 0) m_s[cl] = mval;
    }
    __syncthreads();

    // 3. norm_mix in place on the x tile
#pragma unroll
    for (int it = 0; it < 4; it++) {
      const int cl = (tid >> 4) + 16 * it;
      const half8 h = ld16(&x_s[cl * XS + ch0]);
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; e++) v[e] = (float)h[e];
      ln_row128(v, gmx, bmx, p.eps_mix);
      half8 o;
#pragma unroll
      for (int e = 0; e < 8; e++) o[e] = (half_t)v[e];
      st16(&x_s[cl * XS + ch0], o);
    }
    __syncthreads();

    // 4. emit and gate GEMMs, gate in fp32, fp32 update -> LDS
#pragma unroll
    for (int cs = 0; cs < TM / 32; cs++) {
      f32x16 acc_e, acc_g;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        acc_e[r] = 0.f;
        acc_g[r] = 0.f;
      }
      const int cl = cs * 32 + (lane & 31);
#pragma unroll
      for (int ks = 0; ks < CL / 16; ks++)
        acc_e = mfma32(we[ks], ld16(&x_s[cl * XS + ks * 16 + 8 * (lane >> 5)]), acc_e);
#pragma unroll
      for (int ks = 0; ks < C / 16; ks++)
        acc_g = mfma32(wg[ks], ld16(&n_s[cl * NS + ks * 16 + 8 * (lane >> 5)]), acc_g);
      const float mv = p.out_mask ? m_s[cl] : 1.f;
#pragma unroll
      for (int r4 = 0; r4 < 4; r4++) {
        f32x4 u;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int r = 4 * r4 + e;
          u[e] = acc_e[r] * sigmoidf_fast(acc_g[r]) * mv;
        }
        const int o = 32 * wave + acc_row32(4 * r4, lane);
        *reinterpret_cast<f32x4*>(&o_s[cl * OS + o]) = u;
      }
    }
    __syncthreads();

    // 5. (+ z), one rounding, 16-byte stores of whole cell rows
#pragma unroll
    for (int it = 0; it < 4; it++) {
      const int cl = (tid >> 4) + 16 * it;
      const int pos = pos0 + cl;
      if (pos < L) {
        const f32x4 u0 = *reinterpret_cast<const f32x4*>(&o_s[cl * OS + ch0]);
        const f32x4 u1 = *reinterpret_cast<const f32x4*>(&o_s[cl * OS + ch0 + 4]);
        half8 o;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          float v0 = u0[e], v1 = u1[e];
          if (p.residual) {
            v0 += (float)zr[it][e];
            v1 += (float)zr[it][e + 4];
          }
          o[e] = (half_t)v0;
          o[e + 4] = (half_t)v1;
        }
        st16(p.out + (row_cells + pos) * C + ch0, o);
      }
    }
  }
}

hipError_t launch_epilogue(const EpilogueArgs& a, int grid, hipStream_t s) {
  hipLaunchKernelGGL(tmu_epilogue_kernel, dim3(grid), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace esm
