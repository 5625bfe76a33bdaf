// Kernel (c): norm_mix LayerNorm over the c channels of the channel-major
// contraction output -> proj_emit (MFMA) -> * sigmoid(proj_gate(LN_in(z))) (MFMA)
// [-> * mask] [-> + z], written cell-major.
//
// Persistent, one 8-wave workgroup per CU (two waves per SIMD). proj_emit and
// proj_gate (64 KB) are staged into LDS once and stay there; after that the waves never
// synchronise: each wave owns whole units of 32 cells of one pair row i, cells
// (i, pos0 .. pos0+31), taken in turn from a per-wave sequence (unit
// 8 blockIdx.x + wave + 8 G k), so a CU's units spread over its four SIMDs. Waves 4-7
// stage the weights while waves 0-3 issue their first unit's loads, and all meet at the
// one barrier: the two waves of a SIMD then run their units a staging time apart, so one's
// LayerNorms and GEMMs overlap the other's loads and stores (with every wave starting
// together, each phase ran on all waves at once).
//
// Per unit, in a wave-private 8 KB LDS buffer:
//   1. x[:, i, pos0:pos0+32] (128 channel rows of 64 contiguous bytes) and z's 32 cells
//      (256 contiguous bytes each) arrive as coalesced 16-byte loads;
//   2. x is staged channel-major; ds_read_b64_tr_b16 (gfx950's transposing LDS read: in
//      each 16-lane group, lane j names a 4-element piece P_j and lane n receives
//      P_{4e + n/4}[n % 4], e = 0..3) turns it straight into B-fragments (cell =
//      lane % 32, channels 16 s + 8 (lane / 32) + 0..7, s = 0..7), two reads per
//      fragment, with no 2-byte transposing writes;
//   3. z is staged cell-major over it (16-byte chunks XOR-swizzled per cell) and each
//      lane reads the B-fragment chunks of its cell; z stays staged for the residual;
//   3. both LayerNorms run in registers on the fragments: a lane holds 64 of its
//      cell's 128 channels and its partner lane (lane ^ 32) the other 64, so the
//      statistics are a lane-local sum plus one exchange (fp32 sums from v_dot2_f32_f16);
//   4. D[o][cell] = W_e[o,:] . LN(x)[cell,:] and the gate GEMM on LN(z) with
//      v_mfma_f32_32x32x16_f16, A-fragments read from the LDS-resident weights, two
//      passes of two 32-row output blocks (4 independent accumulator chains each);
//   5. the gate in fp32, the mask, the residual z (each lane's accumulator rows are 4
//      consecutive channels of its cell: one 8-byte piece of the staged z, overwritten
//      in place by the output), one rounding to fp16; stored as whole 256-byte cell
//      rows (16 lanes x 16 B).
// The output gate is recomputed from z rather than stored by kernel (a): z is 2C bytes
// per cell, a stored gate would cost a write plus a read of 2C bytes.
#include "common.h"
#include "kernels.h"

namespace esm {

namespace {
constexpr int C = 128;          // pair channels (output)
constexpr int CL = 128;         // latent channels (contraction output)
constexpr int U = kEpiUnit;     // cells per unit
constexpr int NW = kEpiWaves;   // waves per workgroup (two per SIMD)
static_assert(U == 32, "a unit is one 32-column MFMA tile of cells");
}  // namespace

// Row stride (halfs) of the cell-major staging (z and the output) and of the staged
// weights: 272 bytes, so the 16-byte reads of 16 consecutive rows at one chunk hit 16
// distinct 4-bank groups, and every address is a per-lane base plus an immediate offset
// (an XOR swizzle would need a live address register per chunk).
constexpr int RS = C + 8;
DEV int cs_off(int cell, int k) { return cell * RS + 8 * k; }

// ds_read_b64_tr_b16 of the x tile (channel-major, 64-byte rows of 32 cells): this lane
// names the piece of 4 cells at (channel k0 + j/4, cells n0 + 4 (j % 4)), j = lane % 16;
// it receives x[k0 + e][n0 + lane % 16] for e = 0..3.
DEV half4 tr_read(const half_t* xs, int k0, int n0, int lane) {
  const int j = lane & 15;
  return ds_read_tr16x4(xs + (k0 + (j >> 2)) * U + n0 + 4 * (j & 3));
}

// LayerNorm of one cell's 128 channels held as MFMA B-fragments: this lane holds channels
// 16 s + 8 h + e (s = 0..7, e = 0..7, h = lane / 32), the partner lane (lane ^ 32) the
// other half. Statistics in fp32: sums of the values and of their squares with
// v_dot2_f32_f16 (two exact fp16 products per instruction), a lane-local sum plus one
// exchange, var = E[x^2] - E[x]^2 (ln_scale_shift). gamma / beta come from LDS (fp32).
DEV void ln_frags(half8 (&v)[CL / 16], const float* w, const float* b, float eps, int h) {
  float s = 0.f, q = 0.f;
#pragma unroll
  for (int k = 0; k < CL / 16; k++) dot2_moments(v[k], s, q);
  s += __shfl_xor(s, 32);
  q += __shfl_xor(q, 32);
  float rstd, shift;
  ln_scale_shift(s, q, 1.0f / CL, eps, rstd, shift);
#pragma unroll
  for (int k = 0; k < CL / 16; k++) {
    const int c0 = 16 * k + 8 * h;
    const f32x4 w0 = *reinterpret_cast<const f32x4*>(w + c0), w1 = *reinterpret_cast<const f32x4*>(w + c0 + 4);
    const f32x4 b0 = *reinterpret_cast<const f32x4*>(b + c0), b1 = *reinterpret_cast<const f32x4*>(b + c0 + 4);
#pragma unroll
    for (int e = 0; e < 4; e++) {
      v[k][e] = ln_value(v[k][e], rstd, shift, w0[e], b0[e]);
      v[k][e + 4] = ln_value(v[k][e + 4], rstd, shift, w1[e], b1[e]);
    }
  }
}

// The staging buffer is private to the wave and a wave's LDS operations complete in
// order; this only keeps the compiler from moving LDS accesses across a phase boundary.
DEV void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <bool USE_MASK, bool RESIDUAL>
__global__ __launch_bounds__(NW * 64, 1) void tmu_epilogue_kernel(EpilogueArgs p) {
  __shared__ __align__(16) half_t w_s[2 * C * RS];     // proj_emit rows, then proj_gate rows
  __shared__ __align__(16) half_t b_s[NW][U * RS];     // per-wave staging: x, then z, then the output
  static_assert(CL * U <= U * RS, "the channel-major x tile fits the staging buffer");
  __shared__ __align__(16) float lnp_s[4][C];          // ln_in w, b; ln_mix w, b

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: keeps descriptors scalar
  const int L = p.L;
  const int h = lane >> 5, cell = lane & 31;
  constexpr bool use_mask = USE_MASK;  // out_mask with a mask: the update is multiplied by it

  // Weights and LayerNorm parameters into LDS once (coalesced 16-byte rounds), by waves 4-7.
  constexpr int NST = (NW / 2) * 64;  // staging threads
  auto stage_weights = [&]() {
    const int ts = tid - NST;
    RowStage<C, NST> re, rg;
    re.load(p.w_emit, ts);
    rg.load(p.w_gate, ts);
    if (ts < C) {
      lnp_s[0][ts] = p.ln_in_w[ts];
      lnp_s[1][ts] = p.ln_in_b[ts];
      lnp_s[2][ts] = p.ln_mix_w[ts];
      lnp_s[3][ts] = p.ln_mix_b[ts];
    }
#pragma unroll
    for (int k = 0; k < RowStage<C, NST>::kPer; k++) {
      const int qq = ts + NST * k, r = qq >> 4, j = qq & 15;
      st16(w_s + r * RS + 8 * j, re.v[k]);
      st16(w_s + (C + r) * RS + 8 * j, rg.v[k]);
    }
  };
  const half_t* we_s = w_s;
  const half_t* wg_s = w_s + C * RS;
  half_t* bs = b_s[wave];

  // One unit's global loads: z (4 cells x 256 B per instruction), x (16 channel rows x
  // 64 B per instruction), the mask. Lanes past L, and a unit past the end, read nothing.
  struct UnitLoads {
    half8 z[8], x[8];
    float m;
  };
  auto unit_coords = [&](int u, int& bi, int& i, int& pos0) {
    const int bl = u / p.tiles_per_line;
    pos0 = (u - bl * p.tiles_per_line) * U;
    bi = bl / L;
    i = bl - bi * L;
  };
  auto load_unit = [&](int u, UnitLoads& ld) {
    const bool live = u < p.ntiles;
    int bi, i, pos0;
    unit_coords(live ? u : 0, bi, i, pos0);
    const size_t row_cells = ((size_t)bi * L + i) * L + pos0;  // first cell of the unit
    const rsrc_t rz = make_rsrc(p.z + row_cells * C);
#pragma unroll
    for (int m = 0; m < 8; m++) {
      const int c = 4 * m + (lane >> 4);
      ld.z[m] = bload16(rz, live && pos0 + c < L ? (uint32_t)(c * C + (lane & 15) * 8) * 2u : kOOB);
    }
    const int q = lane & 3;
    const bool okx = live && pos0 + 8 * q < p.ldx;
#pragma unroll
    for (int m = 0; m < 8; m++) {
      const rsrc_t rx = make_rsrc(p.x + (((size_t)bi * CL + 16 * m) * L + i) * p.ldx + pos0);
      ld.x[m] = bload16(rx, okx ? (uint32_t)((size_t)(lane >> 2) * L * p.ldx + 8 * q) * 2u : kOOB);
    }
    ld.m = 1.f;
    if (use_mask) {
      const rsrc_t rm = make_rsrc(p.mask + row_cells);
      ld.m = h2f(bload2(rm, live && pos0 + cell < L ? (uint32_t)cell * 2u : kOOB));
    }
  };

  auto process_unit = [&](int u, const UnitLoads& ld) {
    int bi, i, pos0;
    unit_coords(u, bi, i, pos0);
    const size_t row_cells = ((size_t)bi * L + i) * L + pos0;  // first cell of the unit
    const int q = lane & 3;
    const float mv = ld.m;
    // 2. x: stage channel-major (64-byte rows), transposing reads into B-fragments.
#pragma unroll
    for (int m = 0; m < 8; m++) st16(&bs[(16 * m + (lane >> 2)) * U + 8 * q], ld.x[m]);
    wave_lds_fence();
    half8 nx[CL / 16];
    const int n0 = 16 * ((lane >> 4) & 1);
#pragma unroll
    for (int s = 0; s < CL / 16; s++) {
      const half4 lo = tr_read(bs, 16 * s + 8 * h, n0, lane);
      const half4 hi = tr_read(bs, 16 * s + 8 * h + 4, n0, lane);
#pragma unroll
      for (int e = 0; e < 4; e++) {
        nx[s][e] = lo[e];
        nx[s][e + 4] = hi[e];
      }
    }
    wave_lds_fence();

    // 3. z: stage cell-major over x, read the B-fragment chunks of this lane's cell. z
    //    stays staged for the residual: the output piece of each lane overwrites exactly
    //    the z piece it adds.
#pragma unroll
    for (int m = 0; m < 8; m++) st16(&bs[cs_off(4 * m + (lane >> 4), lane & 15)], ld.z[m]);
    wave_lds_fence();
    half8 nz[CL / 16];
#pragma unroll
    for (int s = 0; s < C / 16; s++) nz[s] = ld16(&bs[cs_off(cell, 2 * s + h)]);

    // 4. LayerNorms in registers.
    ln_frags(nz, lnp_s[0], lnp_s[1], p.eps_in, h);
    ln_frags(nx, lnp_s[2], lnp_s[3], p.eps_mix, h);

    // 5. GEMMs, two passes of two 32-row output blocks; gate, mask, residual, one
    //    rounding; 8-byte pieces staged cell-major.
#pragma unroll
    for (int pass = 0; pass < 2; pass++) {
      f32x16 e[2], g[2];
#pragma unroll
      for (int t = 0; t < 2; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          e[t][r] = 0.f;
          g[t][r] = 0.f;
        }
      // A-fragments read per k-step (the other wave on the SIMD covers their latency); the
      // scheduling barrier keeps the compiler from hoisting every k-step's reads at once.
#pragma unroll
      for (int s = 0; s < CL / 16; s++) {
        half8 wa[2][2];  // [t][emit, gate]
#pragma unroll
        for (int t = 0; t < 2; t++) {
          const int o = 32 * (2 * pass + t) + cell;
          wa[t][0] = ld16(we_s + o * RS + 8 * (2 * s + h));
          wa[t][1] = ld16(wg_s + o * RS + 8 * (2 * s + h));
        }
#pragma unroll
        for (int t = 0; t < 2; t++) {
          e[t] = mfma32(wa[t][0], nx[s], e[t]);
          g[t] = mfma32(wa[t][1], nz[s], g[t]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int t = 0; t < 2; t++) {
        const int ob = 2 * pass + t;
#pragma unroll
        for (int j = 0; j < 4; j++) {
          // channels 32 ob + 8 j + 4 h + 0..3 of this lane's cell: the rows its
          // accumulators hold, and one 8-byte piece of the staged z
          half4* piece = reinterpret_cast<half4*>(&bs[cs_off(cell, 4 * ob + j) + 4 * h]);
          const half4 zr = *piece;
          half4 o;
#pragma unroll
          for (int r = 0; r < 4; r++) {
            float v = e[t][4 * j + r] * sigmoid_from_t(g[t][4 * j + r] * kNegLog2e);
            if (use_mask) v *= mv;
            if (RESIDUAL) v += (float)zr[r];
            o[r] = (half_t)v;
          }
          *piece = o;
        }
      }
    }
    wave_lds_fence();

    // 6. Whole 256-byte cell rows: 16 lanes x 16 B, 4 cells per store.
    const rsrc_t ro = make_rsrc(p.out + row_cells * C);
#pragma unroll
    for (int m = 0; m < 8; m++) {
      const int c = 4 * m + (lane >> 4);
      bstore16(ro, pos0 + c < L ? (uint32_t)(c * C + (lane & 15) * 8) * 2u : kOOB, ld16(&bs[cs_off(c, lane & 15)]));
    }
    wave_lds_fence();
  };

  // Consecutive units go to the waves of one workgroup: the two 32-cell halves of a
  // 128-byte line of x are then read on one CU (dealt to different XCDs, each half
  // fetched the whole line again: 1.8x the compulsory reads). At 8 units per pair row a
  // workgroup's units are one whole row of x per channel; rows are not line-aligned
  // (ld = 240: 480 bytes), so the line at the end of row i is also the start of row i + 1,
  // and the XCD-aware order puts consecutive rows on one XCD, whose L2 then fetches that
  // line once.
  // Every wave passes the one barrier once: waves 0-3 with their first unit's loads in
  // flight, waves 4-7 after the staging.
  const int G = gridDim.x;
  int u = xcd_remap(blockIdx.x, G) * NW + wave;
  if (wave < NW / 2) {
    UnitLoads ld;
    load_unit(u, ld);
    __syncthreads();
    if (u < p.ntiles) process_unit(u, ld);
  } else {
    stage_weights();
    __syncthreads();
    if (u < p.ntiles) {
      UnitLoads ld;
      load_unit(u, ld);
      process_unit(u, ld);
    }
  }
  for (u += G * NW; u < p.ntiles; u += G * NW) {
    UnitLoads ld;
    load_unit(u, ld);
    process_unit(u, ld);
  }
}

hipError_t launch_epilogue(const EpilogueArgs& a, int grid, hipStream_t s) {
  const bool m = a.out_mask && a.mask;
  if (m && a.residual)
    ESM_LAUNCH((tmu_epilogue_kernel<true, true>), dim3(grid), dim3(NW * 64), 0, s, a);
  else if (m)
    ESM_LAUNCH((tmu_epilogue_kernel<true, false>), dim3(grid), dim3(NW * 64), 0, s, a);
  else if (a.residual)
    ESM_LAUNCH((tmu_epilogue_kernel<false, true>), dim3(grid), dim3(NW * 64), 0, s, a);
  else
    ESM_LAUNCH((tmu_epilogue_kernel<false, false>), dim3(grid), dim3(NW * 64), 0, s, a);
  return hipGetLastError();
}

}  // namespace esm
