// Kernel (c): norm_mix LayerNorm over the c channels of the channel-major
// contraction output -> proj_emit (MFMA) -> * sigmoid(proj_gate(LN_in(z))) (MFMA)
// [-> * mask] [-> + z], written cell-major.
//
// Persistent like kernel (a): one 8-wave workgroup per CU (2 waves per SIMD). Wave w
// owns output channels [32 (w%4), +32) for cells [32 (w/4), +32) of each tile and keeps
// those rows of proj_emit and proj_gate in VGPRs as MFMA A-fragments. A tile is 64
// cells of one row i of the pair grid, cells (i, pos0..pos0+63). Per tile:
//   1. x[:, i, pos0:pos0+64] arrives as 128 channel rows of 128 contiguous bytes and
//      is transposed into an LDS tile [cell][c]; its 16-byte chunks are XOR-swizzled
//      per row so both the transposing 2-byte writes and the 16-byte MFMA reads are
//      free of bank conflicts;
//   2. z's 64 cells (256 contiguous bytes each) are LayerNormed (norm_start) into a
//      second tile; the raw z stays in registers for the residual;
//   3. norm_mix is applied in place to the x tile (fp32 statistics);
//   4. D[o][cell] = W_e[o,:] . LN(x)[cell,:] and the gate GEMM on LN(z) with
//      v_mfma_f32_32x32x16_f16, each split over two K halves so 4 accumulator chains
//      keep the MFMA pipe full; each lane holds groups of 4 consecutive output channels
//      of one cell, applies the gate in fp32 and stages the fp32 update in LDS;
//   5. the update plus z is rounded once and leaves as whole 256-byte cell rows
//      (scattered 32-byte pieces of rows measured 2x slower).
// The input tiles are double-buffered; a tile costs three barriers. The output gate
// is recomputed from z rather than stored by kernel (a): z is 2C bytes per cell, a
// stored gate would cost a write plus a read of 2C bytes.
#include "common.h"
#include "kernels.h"

namespace esm {

namespace {
constexpr int C = 128;          // pair channels (output)
constexpr int CL = 128;         // latent channels (contraction output)
constexpr int TM = kCellTile;   // cells per tile
constexpr int XS = CL;          // LDS row stride (halfs), x tile (swizzled, no padding)
constexpr int NS = C + 8;       // LDS row stride (halfs), LN(z) tile
constexpr int OS = C;           // LDS row stride (floats), update staging (swizzled)
constexpr int NW = 8;           // waves per workgroup
constexpr int OPW = 32;         // output channels per wave (one 32-row MFMA tile)
constexpr int CPT = TM * 16 / (NW * 64);         // cells LayerNormed per thread per tile
constexpr int XPT = CL * (TM / 8) / (NW * 64);   // 16-byte x chunks per thread per tile
static_assert(C / OPW * (TM / 32) == NW && CPT == 2 && XPT == 2, "tile split assumed below");
}  // namespace

// Physical 16-byte chunk of logical chunk k in row r of the x tile. Rows 8q+e with a
// fixed e (one transposing write instruction) land in 8 distinct chunks, and 16
// consecutive rows (one MFMA fragment read) in 16 distinct chunks.
DEV int xs_chunk(int row, int k) {
  const int f = 2 * ((row & 7) ^ ((row >> 4) & 3)) + ((row >> 3) & 1);
  return k ^ f;
}

// Float offset of (cell, channel o) in the fp32 update staging tile: 16-byte chunk o/4
// stored at chunk (o/4) ^ (cell & 15), so the 16-byte writes of 16 consecutive cells hit
// 16 distinct bank groups.
DEV int os_off(int cell, int o) { return cell * OS + 4 * ((o >> 2) ^ (cell & 15)) + (o & 3); }

template <bool USE_MASK>
__global__ __launch_bounds__(NW * 64, 1) void tmu_epilogue_kernel(EpilogueArgs p) {
  __shared__ __align__(16) half_t x_s[2][TM * XS];
  __shared__ __align__(16) half_t n_s[2][TM * NS];
  __shared__ __align__(16) float o_s[TM * OS];
  __shared__ __align__(16) float m_s[2][TM];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: keeps descriptors scalar
  const int L = p.L;
  constexpr bool use_mask = USE_MASK;  // out_mask with a mask: the update is multiplied by it

  // Weight A-fragments: row = output channel o = 32 og + lane%32, k = 16 ks + 8 (lane/32) + e.
  const int og = wave & 3, chalf = wave >> 2;
  // proj_emit, then proj_gate, stream through LDS (the fp32 staging tile, 32 KB, is free
  // until the first tile's GEMMs, two barriers into the loop) in coalesced rounds; both
  // rounds' loads are in flight together.
  half8 we[CL / 16], wg[C / 16];
  auto load_weights = [&] {
    static_assert(C * CL * 2 <= TM * OS * 4 && C * C * 2 <= TM * OS * 4, "a weight fits the staging tile");
    half_t* w_s = reinterpret_cast<half_t*>(o_s);
    RowStage<C, NW * 64> r0, r1;
    r0.load(p.w_emit, tid);
    r1.load(p.w_gate, tid);
    const int o = OPW * og + (lane & 31);
    r0.store(w_s, tid);
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < CL / 16; ks++) we[ks] = staged_chunk(w_s, o, 2 * ks + (lane >> 5));
    __syncthreads();
    r1.store(w_s, tid);
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < C / 16; ks++) wg[ks] = staged_chunk(w_s, o, 2 * ks + (lane >> 5));
  };
  const int ch0 = (lane & 15) * 8;
  float gin[8], bin[8], gmx[8], bmx[8];
#pragma unroll
  for (int e = 0; e < 8; e++) {
    gin[e] = p.ln_in_w[ch0 + e];
    bin[e] = p.ln_in_b[ch0 + e];
    gmx[e] = p.ln_mix_w[ch0 + e];
    bmx[e] = p.ln_mix_b[ch0 + e];
  }

  auto coords = [&](int tile, int& bi, int& i, int& pos0) {
    const int bl = tile / p.tiles_per_line;
    pos0 = (tile - bl * p.tiles_per_line) * TM;
    bi = bl / L;
    i = bl - bi * L;
  };

  // Issue one tile's loads: x rows (channel d, 8 positions per chunk), z cells and, with
  // out_mask, the raw mask. Out-of-range lanes, and the tile past the end that the
  // pipeline's last prefetch names, read nothing.
  auto load_tile = [&](int tile, half8 (&xq)[XPT], half8 (&zq)[CPT], uint16_t (&mq)[CPT]) {
    const bool live = tile < p.ntiles;
    int bi, i, pos0;
    coords(live ? tile : 0, bi, i, pos0);
    const size_t row_cells = ((size_t)bi * L + i) * L;
    const int q = lane & 7;
    const bool okx = live && pos0 + q * 8 < L;
#pragma unroll
    for (int u = 0; u < XPT; u++) {
      // this wave's lanes cover channels d = 64u + 8 wave + (lane >> 3), 8 positions each
      const rsrc_t rx = make_rsrc(p.x + (((size_t)bi * CL + 64 * u + 8 * wave) * L + i) * p.ldx + pos0);
      xq[u] = bload16(rx, okx ? (uint32_t)((size_t)(lane >> 3) * L * p.ldx + q * 8) * 2u : kOOB);
    }
    const rsrc_t rz = make_rsrc(p.z + (row_cells + pos0) * C);
    const rsrc_t rm = make_rsrc(use_mask ? (const void*)(p.mask + row_cells + pos0) : (const void*)p.z);
    (void)rm;
#pragma unroll
    for (int it = 0; it < CPT; it++) {
      const int cl = (tid >> 4) + (NW * 4) * it;
      const bool ok = live && pos0 + cl < L;
      zq[it] = bload16(rz, ok ? (uint32_t)(cl * C + ch0) * 2u : kOOB);
      if (use_mask) mq[it] = bload2(rm, ok ? (uint32_t)cl * 2u : kOOB);
    }
  };

  auto process_tile = [&](int tile, const half8 (&xq)[XPT], const half8 (&zq)[CPT], const uint16_t (&mq)[CPT],
                          int nb) {
    int bi, i, pos0;
    coords(tile, bi, i, pos0);
    const size_t row_cells = ((size_t)bi * L + i) * L;
    half_t* xs = x_s[nb];
    half_t* ns = n_s[nb];
    // 1. x chunks -> LDS [cell][d], transposed, swizzled
#pragma unroll
    for (int u = 0; u < XPT; u++) {
      const int d = (tid >> 3) + 64 * u, q = tid & 7;
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const int row = q * 8 + e;
        xs[row * XS + 8 * xs_chunk(row, d >> 3) + (d & 7)] = xq[u][e];
      }
    }
    // 2. LN_in(z) -> LDS (the raw z stays in registers for the residual)
#pragma unroll
    for (int it = 0; it < CPT; it++) {
      const int cl = (tid >> 4) + (NW * 4) * it;
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; e++) v[e] = (float)zq[it][e];
      ln_row128(v, gin, bin, p.eps_in);
      half8 o;
#pragma unroll
      for (int e = 0; e < 8; e++) o[e] = (half_t)v[e];
      st16(&ns[cl * NS + ch0], o);
      if ((lane & 15) == 0) m_s[nb][cl] = use_mask ? h2f(mq[it]) : 1.f;
    }
    __syncthreads();

    // 3. norm_mix in place on the x tile (lane reads logical chunk lane%16 of its cell)
#pragma unroll
    for (int it = 0; it < CPT; it++) {
      const int cl = (tid >> 4) + (NW * 4) * it;
      half_t* px = &xs[cl * XS + 8 * xs_chunk(cl, lane & 15)];
      const half8 h = ld16(px);
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; e++) v[e] = (float)h[e];
      ln_row128(v, gmx, bmx, p.eps_mix);
      half8 o;
#pragma unroll
      for (int e = 0; e < 8; e++) o[e] = (half_t)v[e];
      st16(px, o);
    }
    __syncthreads();

    // 4. emit and gate GEMMs for this wave's 32 cells and 32 output channels, each K split
    //    in two (4 independent accumulator chains); gate in fp32; fp32 update -> LDS
    {
      const int cell = 32 * chalf + (lane & 31);
      f32x16 e0, e1, g0, g1;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        e0[r] = 0.f;
        e1[r] = 0.f;
        g0[r] = 0.f;
        g1[r] = 0.f;
      }
#pragma unroll
      for (int ks = 0; ks < CL / 32; ks++) {
        const int k1 = ks + CL / 32;
        e0 = mfma32(we[ks], ld16(&xs[cell * XS + 8 * xs_chunk(cell, 2 * ks + (lane >> 5))]), e0);
        e1 = mfma32(we[k1], ld16(&xs[cell * XS + 8 * xs_chunk(cell, 2 * k1 + (lane >> 5))]), e1);
        g0 = mfma32(wg[ks], ld16(&ns[cell * NS + 16 * ks + 8 * (lane >> 5)]), g0);
        g1 = mfma32(wg[k1], ld16(&ns[cell * NS + 16 * k1 + 8 * (lane >> 5)]), g1);
      }
      const float mv = m_s[nb][cell];
#pragma unroll
      for (int r4 = 0; r4 < 4; r4++) {
        f32x4 u;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int r = 4 * r4 + e;
          u[e] = (e0[r] + e1[r]) * sigmoidf_fast(g0[r] + g1[r]) * mv;
        }
        *reinterpret_cast<f32x4*>(&o_s[os_off(cell, OPW * og + acc_row32(4 * r4, lane))]) = u;
      }
    }
    __syncthreads();

    // 5. (+ z from registers), one rounding, whole 256-byte cell rows (16 lanes x 16 B);
    //    cells past L are dropped by the buffer range check.
    const rsrc_t ro = make_rsrc(p.out + (row_cells + pos0) * C);
#pragma unroll
    for (int it = 0; it < CPT; it++) {
      const int cl = (tid >> 4) + (NW * 4) * it;
      const f32x4 u0 = *reinterpret_cast<const f32x4*>(&o_s[os_off(cl, ch0)]);
      const f32x4 u1 = *reinterpret_cast<const f32x4*>(&o_s[os_off(cl, ch0 + 4)]);
      half8 o;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        float v0 = u0[e], v1 = u1[e];
        if (p.residual) {
          v0 += (float)zq[it][e];
          v1 += (float)zq[it][e + 4];
        }
        o[e] = (half_t)v0;
        o[e + 4] = (half_t)v1;
      }
      bstore16(ro, pos0 + cl < L ? (uint32_t)(cl * C + ch0) * 2u : kOOB, o);
    }
  };

  // Software pipeline: the next tile's loads fly while this one computes (ping-pong
  // register buffers, unrolled by two so no register copy waits on a load).
  const int G = gridDim.x;
  half8 xA[XPT], zA[CPT], xB[XPT], zB[CPT];
  uint16_t mA[CPT] = {}, mB[CPT] = {};
  int tile = blockIdx.x;
  load_tile(tile, xA, zA, mA);  // the first tile's data goes out before the weights
  load_weights();
  for (; tile < p.ntiles; tile += 2 * G) {
    load_tile(tile + G, xB, zB, mB);
    process_tile(tile, xA, zA, mA, 0);
    if (tile + G >= p.ntiles) break;
    load_tile(tile + 2 * G, xA, zA, mA);
    process_tile(tile + G, xB, zB, mB, 1);
  }
}

hipError_t launch_epilogue(const EpilogueArgs& a, int grid, hipStream_t s) {
  if (a.out_mask && a.mask)
    hipLaunchKernelGGL(tmu_epilogue_kernel<true>, dim3(grid), dim3(NW * 64), 0, s, a);
  else
    hipLaunchKernelGGL(tmu_epilogue_kernel<false>, dim3(grid), dim3(NW * 64), 0, s, a);
  return hipGetLastError();
}

}  // namespace esm
