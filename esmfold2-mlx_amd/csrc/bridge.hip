// Kernel (c+a): the middle of a TMU pair (outgoing then incoming, C = c = 128) in one launch:
//   z1 = z + (LN_mix(x) W_e^T) * sigmoid(LN_in(z) W_g^T)        the outgoing update's kernel (c)
//   a', b' = gate(LN_in'(z1) W'^T) * mask, incoming layout         the incoming update's kernel (a)
// z1 is produced and consumed on chip: the pair runs in five launches instead of six and
// the residual stream is written once (as z1) between the two contractions.
//
// Persistent, one 8-wave workgroup per CU (two waves per SIMD), over blocks of 8 x 8 cells
// (rows i0 .. i0+7, columns j0 .. j0+7). Two cell orders are used inside a tile:
//   x-order  xo = 8 di + dj   the order of x's rows (16 bytes of x hold dj = 0..7);
//   k-order  kc = 8 dj + di   the incoming operands' order (operand row j0 + dj, k = i0 + di:
//                             one staged channel row is one 128-byte fragment segment).
// Per tile:
//   P1  x (128 channel rows x 8 rows of 16 bytes), z (64 cells of 256 bytes) and the mask
//       arrive as coalesced loads issued one tile ahead; x is staged channel-major, z in
//       x-order rows;                                                            barrier
//   P2  the mask staged (k-order); waves 0-3 LayerNorm x (ds_read_b64_tr_b16 turns
//       channel-major pieces into 4 channels of one cell per lane), waves 4-7 LayerNorm z;
//       4 lanes per cell, fp32 statistics (v_dot2_f32_f16 sums); results in x-order rows;
//                                                                                barrier
//   P3  wave w: outputs 16 w .. 16 w+15 of the emit and gate GEMMs for all 64 cells
//       (v_mfma_f32_16x16x32_f16, weights in registers), gate, residual, one rounding:
//       z1 in x-order rows;                                                      barrier
//   P4  z1 leaves as whole 256-byte cells; LN_in'(z1) per cell (16 lanes) into k-order
//       rows;                                                                    barrier
//   P5  the incoming projection as kernel (a) runs it (bundle in registers, 32x32x16
//       MFMAs, gate and mask in fp32), staged per channel, stored as one 128-byte segment
//       of a fragment tile per channel.
// The workgroup order is XCD-aware: consecutive tiles (the 8 along a row that share each
// 128-byte line of x) run on one L2.
#include "common.h"
#include "kernels.h"

namespace esm {

namespace {
constexpr int C = 128;            // pair channels
constexpr int CL = 128;           // latent channels
constexpr int NW = 8;             // waves per workgroup
constexpr int NT = NW * 64;
constexpr int TC = 64;            // cells per tile (8 x 8)
constexpr int NS = C + 8;         // LDS row stride (halfs) of the cell-row tiles: 272 B
// Channel-major x tile: rows of 64 cells + 16 halfs (160 B = 40 banks). The transposing
// reads of one half-wave touch 8 consecutive rows at one column: 8 x 40 mod 64 banks are 8
// disjoint 8-bank groups.
constexpr int XS = TC + 16;
constexpr int CPW = 32;           // incoming channels (of a or of b) per wave
// LDS carve (bytes): x tile, later the z1 tile; raw z; LN_mix(x); LN_in(z), later LN_in'(z1);
// per-wave output staging. The start-up weight staging (64 KB rounds) uses the same bytes.
constexpr int X_B = CL * XS * 2, R_B = TC * NS * 2, ST_B = NW * CPW * TC * 2;
constexpr int OFF_Z = X_B, OFF_NX = OFF_Z + R_B, OFF_NZ = OFF_NX + R_B, OFF_ST = OFF_NZ + R_B;
constexpr int SMEM_B = OFF_ST + ST_B;
static_assert(R_B <= X_B, "the z1 tile fits the x tile's place");
static_assert(SMEM_B >= 2 * CL * C * 2, "a 64 KB weight round fits the tile area");
static_assert(TC * 16 == 2 * NT, "two cells per thread in the 16-lane phases");
}  // namespace

// k-order index of an x-order cell.
DEV int br_kc(int xo) { return 8 * (xo & 7) + (xo >> 3); }

// Output staging (as kernel (a)): chunk q of channel row ch at chunk q ^ ((ch >> 1) & 7).
DEV int br_st_off(int ch, int cell) { return ch * TC + 8 * ((cell >> 3) ^ ((ch >> 1) & 7)) + (cell & 7); }

typedef short br_v4s __attribute__((ext_vector_type(4)));
// ds_read_b64_tr_b16 on the channel-major x tile: in each 16-lane group, lane j names the
// 4 cells n0 + 4 (j % 4) .. +3 of channel k0 + j / 4, and lane n receives x[k0 + e][n0 + n],
// e = 0..3 (gfx950's transposing LDS read).
DEV half4 br_tr_read(const half_t* xs, int k0, int n0, int lane) {
  const int j = lane & 15;
  const half_t* p = xs + (k0 + (j >> 2)) * XS + n0 + 4 * (j & 3);
  const br_v4s v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) br_v4s*)(__attribute__((address_space(3))) half_t*)p);
  return __builtin_bit_cast(half4, v);
}

// The sums of a 128-channel row held by 4 lanes (l, l ^ 16, l ^ 32, l ^ 48), to every one of them.
DEV void br_quad_sum(float& s, float& q) {
  s += __shfl_xor(s, 16);
  q += __shfl_xor(q, 16);
  s += __shfl_xor(s, 32);
  q += __shfl_xor(q, 32);
}

// gamma / beta of channels ch0 .. ch0+7 from LDS.
DEV void br_params(const float* w, const float* b, int ch0, float (&g)[8], float (&bb)[8]) {
  const f32x4 w0 = *reinterpret_cast<const f32x4*>(w + ch0), w1 = *reinterpret_cast<const f32x4*>(w + ch0 + 4);
  const f32x4 b0 = *reinterpret_cast<const f32x4*>(b + ch0), b1 = *reinterpret_cast<const f32x4*>(b + ch0 + 4);
#pragma unroll
  for (int e = 0; e < 4; e++) {
    g[e] = w0[e];
    g[e + 4] = w1[e];
    bb[e] = b0[e];
    bb[e + 4] = b1[e];
  }
}

template <bool HAS_MASK>
__global__ __launch_bounds__(NT, 1) void tmu_bridge_kernel(BridgeArgs p) {
  __shared__ __align__(16) char smem[SMEM_B];
  // [0, 1] outgoing LN_in w, b; [2, 3] LN_mix w, b; [4, 5] incoming LN_in w, b
  __shared__ __align__(16) float lnp[6][C];
  __shared__ __align__(16) float m_s[TC];  // mask, k-order
  half_t* xs = reinterpret_cast<half_t*>(smem);            // [ch][xo], stride XS
  half_t* z1s = xs;                                        // [xo][NS] from P3 on
  half_t* zs = reinterpret_cast<half_t*>(smem + OFF_Z);    // [xo][NS]
  half_t* nxs = reinterpret_cast<half_t*>(smem + OFF_NX);  // [xo][NS]
  half_t* nzs = reinterpret_cast<half_t*>(smem + OFF_NZ);  // [xo][NS] in P2-P3, [kc][NS] in P4-P5
  half_t* w_s = reinterpret_cast<half_t*>(smem);           // start-up only

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: keeps descriptors scalar
  const int l16 = lane & 15, q4 = lane >> 4;
  const int L = p.L, tpd = p.tpd;
  const size_t plane_h = (size_t)p.rbn * p.kbn * FragLayout::kTileHalfs;

  // Incoming bundle: wave w keeps 32 channels of a (waves 0-3) or b (waves 4-7), signal and
  // gate rows, as 32x32x16 B-fragments (column = channel, k = 16 ks + 8 (lane / 32) + e).
  // Outgoing emit / gate: wave w keeps rows 16 w .. 16 w+15 as 16x16x32 A-fragments
  // (row = lane % 16, k = 32 ks + 8 (lane / 16) + e).
  const int is_b = wave >= NW / 2;
  const int ch_base = CPW * (wave - is_b * (NW / 2));
  half8 ws[C / 16], wg[C / 16], we16[C / 32], wg16[C / 32];
  auto load_weights = [&] {
    RowStage<2 * CL, NT> r0, r1;
    RowStage<C, NT> re, rg;
    r0.load(p.w_bundle, tid);               // signal rows [s_a | s_b]
    r1.load(p.w_bundle + 2 * CL * C, tid);  // gate rows [g_a | g_b]
    re.load(p.w_emit, tid);
    rg.load(p.w_gate, tid);
    if (tid < C) {
      lnp[0][tid] = p.lno_w[tid];
      lnp[1][tid] = p.lno_b[tid];
      lnp[2][tid] = p.lnm_w[tid];
      lnp[3][tid] = p.lnm_b[tid];
      lnp[4][tid] = p.lni_w[tid];
      lnp[5][tid] = p.lni_b[tid];
    }
    const int row = is_b * CL + ch_base + (lane & 31);
    r0.store(w_s, tid);
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < C / 16; ks++) ws[ks] = staged_chunk(w_s, row, 2 * ks + (lane >> 5));
    __syncthreads();
    r1.store(w_s, tid);
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < C / 16; ks++) wg[ks] = staged_chunk(w_s, row, 2 * ks + (lane >> 5));
    __syncthreads();
    re.store(w_s, tid);
    rg.store(w_s + C * 128, tid);
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < C / 32; ks++) {
      we16[ks] = staged_chunk(w_s, 16 * wave + l16, 4 * ks + q4);
      wg16[ks] = staged_chunk(w_s + C * 128, 16 * wave + l16, 4 * ks + q4);
    }
    __syncthreads();
  };

  auto coords = [&](int tile, int& bi, int& i0, int& j0) {
    bi = tile / (tpd * tpd);
    const int t = tile - bi * tpd * tpd, ti = t / tpd;
    i0 = 8 * ti;
    j0 = 8 * (t - ti * tpd);
  };
  struct TileLoads {
    half8 z[2], x[2];
    uint16_t m;
  };
  const rsrc_t rz = make_rsrc(p.z), rx = make_rsrc(p.x), rz1 = make_rsrc(p.z1);
  const rsrc_t rm = make_rsrc(HAS_MASK ? (const void*)p.mask : (const void*)p.z);
  // One tile's loads; cells outside the grid and a tile past the end read nothing (zeros).
  auto load_tile = [&](int tile, TileLoads& tl) {
    const bool live = tile < p.ntiles;
    int bi, i0, j0;
    coords(live ? tile : 0, bi, i0, j0);
#pragma unroll
    for (int it = 0; it < 2; it++) {
      const int xo = (tid >> 4) + 32 * it, di = xo >> 3, dj = xo & 7;
      const bool ok = live && i0 + di < L && j0 + dj < L;
      const uint32_t cell = (uint32_t)(((size_t)bi * L + i0 + di) * L + j0 + dj);
      tl.z[it] = bload16(rz, ok ? (cell * C + 8 * l16) * 2u : kOOB);
    }
#pragma unroll
    for (int u = 0; u < 2; u++) {
      const int id = tid + NT * u, ch = id >> 3, di = id & 7;
      const bool ok = live && i0 + di < L;
      const size_t off = (((size_t)bi * CL + ch) * L + i0 + di) * p.ldx + j0;
      tl.x[u] = bload16(rx, ok ? (uint32_t)(off * 2u) : kOOB);
    }
    tl.m = 0;
    if (HAS_MASK) {
      const int kc = tid & 63, di = kc & 7, dj = kc >> 3;
      const bool ok = live && tid < TC && i0 + di < L && j0 + dj < L;
      tl.m = bload2(rm, ok ? (uint32_t)((((size_t)bi * L + i0 + di) * L + j0 + dj) * 2u) : kOOB);
    }
  };

  auto process_tile = [&](int tile, const TileLoads& tl) {
    int bi, i0, j0;
    coords(tile, bi, i0, j0);
    // P1: x channel-major (xo = 8 di + dj), z in x-order rows.
#pragma unroll
    for (int u = 0; u < 2; u++) {
      const int id = tid + NT * u, ch = id >> 3, di = id & 7;
      st16(&xs[ch * XS + 8 * di], tl.x[u]);
    }
#pragma unroll
    for (int it = 0; it < 2; it++) st16(&zs[((tid >> 4) + 32 * it) * NS + 8 * l16], tl.z[it]);
    __syncthreads();
    // (the mask is staged after the barrier: until then other waves may still read the
    // previous tile's mask in P5)
    if (HAS_MASK && tid < TC) m_s[tid] = h2f(tl.m);

    // P2: LN_mix(x) on waves 0-3, LN_in(z) on waves 4-7; lane (g = lane / 16, n = lane % 16)
    // of wave w holds cell xo = 16 (w % 4) + n. Cells outside the grid become zero rows.
    // A cell outside the grid gets whatever its zero input gives: its column of the P3
    // GEMMs is its own, and its z1 is never stored.
    {
      const int xo = 16 * (wave & 3) + l16;
      float s = 0.f, q = 0.f, rstd, shift;
      if (wave < NW / 2) {
        half4 h[8];
#pragma unroll
        for (int t = 0; t < 8; t++) {
          h[t] = br_tr_read(xs, 4 * (q4 + 4 * t), 16 * wave, lane);
          dot2_moments(h[t], s, q);
        }
        br_quad_sum(s, q);
        ln_scale_shift(s, q, 1.0f / 128.0f, p.lnm_eps, rstd, shift);
#pragma unroll
        for (int t = 0; t < 8; t++) {
          const int c0 = 4 * (q4 + 4 * t);
          const f32x4 gw = *reinterpret_cast<const f32x4*>(&lnp[2][c0]);
          const f32x4 gb = *reinterpret_cast<const f32x4*>(&lnp[3][c0]);
          half4 o;
#pragma unroll
          for (int e = 0; e < 4; e++) o[e] = ln_value(h[t][e], rstd, shift, gw[e], gb[e]);
          *reinterpret_cast<half4*>(&nxs[xo * NS + c0]) = o;
        }
      } else {
        half8 h[4];
#pragma unroll
        for (int t = 0; t < 4; t++) {
          h[t] = ld16(&zs[xo * NS + 8 * (q4 + 4 * t)]);
          dot2_moments(h[t], s, q);
        }
        br_quad_sum(s, q);
        ln_scale_shift(s, q, 1.0f / 128.0f, p.lno_eps, rstd, shift);
#pragma unroll
        for (int t = 0; t < 4; t++) {
          const int c0 = 8 * (q4 + 4 * t);
          half8 o;
#pragma unroll
          for (int e4 = 0; e4 < 8; e4 += 4) {
            const f32x4 gw = *reinterpret_cast<const f32x4*>(&lnp[0][c0 + e4]);
            const f32x4 gb = *reinterpret_cast<const f32x4*>(&lnp[1][c0 + e4]);
#pragma unroll
            for (int e = 0; e < 4; e++) o[e4 + e] = ln_value(h[t][e4 + e], rstd, shift, gw[e], gb[e]);
          }
          st16(&nzs[xo * NS + c0], o);
        }
      }
    }
    __syncthreads();

    // P3: D[o][cell] for o = 16 wave .. +15 and all 64 cells (x-order): a lane holds cell
    // 16 cb + l16, outputs 16 wave + 4 q4 .. +3. Gate in fp32, [mask,] residual, one rounding.
    {
      f32x4 ae[4], ag[4];
#pragma unroll
      for (int cb = 0; cb < 4; cb++) {
        ae[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
        ag[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int ks = 0; ks < C / 32; ks++)
#pragma unroll
        for (int cb = 0; cb < 4; cb++) {
          const int r = (16 * cb + l16) * NS + 32 * ks + 8 * q4;
          ae[cb] = mfma16(we16[ks], ld16(&nxs[r]), ae[cb]);
          ag[cb] = mfma16(wg16[ks], ld16(&nzs[r]), ag[cb]);
        }
      const int o0 = 16 * wave + 4 * q4;
#pragma unroll
      for (int cb = 0; cb < 4; cb++) {
        const int xo = 16 * cb + l16;
        const half4 zr = *reinterpret_cast<const half4*>(&zs[xo * NS + o0]);
        const float mv = HAS_MASK && p.out_mask ? m_s[br_kc(xo)] : 1.f;
        half4 o;
#pragma unroll
        for (int r = 0; r < 4; r++) {
          float v = ae[cb][r] * sigmoid_from_t(ag[cb][r] * kNegLog2e);
          if (HAS_MASK && p.out_mask) v *= mv;
          v += (float)zr[r];
          __asm__ volatile("" : "+v"(v));  // fp32, then one rounding to fp16
          o[r] = (half_t)v;
        }
        *reinterpret_cast<half4*>(&z1s[xo * NS + o0]) = o;
      }
    }
    __syncthreads();

    // P4: z1 out as whole cells; LN_in'(z1) (16 lanes per cell) into k-order rows.
    // Cells outside the grid (only in the last tile row or column) become zero rows, so
    // that k past L is exactly zero in the incoming operands.
    const int ch0 = 8 * l16;
    const bool edge = i0 + 8 > L || j0 + 8 > L;
#pragma unroll
    for (int it = 0; it < 2; it++) {
      const int xo = (tid >> 4) + 32 * it, di = xo >> 3, dj = xo & 7;
      const bool in = i0 + di < L && j0 + dj < L;
      const half8 zv = ld16(&z1s[xo * NS + ch0]);
      const uint32_t cell = (uint32_t)(((size_t)bi * L + i0 + di) * L + j0 + dj);
      bstore16(rz1, in ? (cell * C + ch0) * 2u : kOOB, zv);
      float g[8], bb[8];
      br_params(lnp[4], lnp[5], ch0, g, bb);
      half8 o = ln_row128_h(zv, g, bb, p.lni_eps);
      if (edge && !in) o = zero_half8();
      st16(&nzs[br_kc(xo) * NS + ch0], o);
    }
    __syncthreads();

    // P5: the incoming projection, D[kc][channel] with both 32-cell halves (4 accumulator
    // chains), gate and mask in fp32, groups of 4 consecutive cells of one channel staged.
    half_t* st = reinterpret_cast<half_t*>(smem + OFF_ST) + wave * CPW * TC;
    f32x16 as[2], ag[2];
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        as[h][r] = 0.f;
        ag[h][r] = 0.f;
      }
#pragma unroll
    for (int ks = 0; ks < C / 16; ks++) {
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const half8 af = ld16(&nzs[(32 * h + (lane & 31)) * NS + 16 * ks + 8 * (lane >> 5)]);
        as[h] = mfma32(af, ws[ks], as[h]);
        ag[h] = mfma32(af, wg[ks], ag[h]);
      }
    }
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
      for (int r4 = 0; r4 < 4; r4++) {
        const int c4 = 32 * h + acc_row32(4 * r4, lane);  // first of 4 consecutive k-order cells
        // (a cell outside the grid has a zero row, so its signal is 0)
        const f32x4 m4 = HAS_MASK ? *reinterpret_cast<const f32x4*>(&m_s[c4]) : f32x4{1.f, 1.f, 1.f, 1.f};
        half4 v;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          float t = as[h][4 * r4 + e] * sigmoidf_fast(ag[h][4 * r4 + e]);
          if (HAS_MASK) t *= m4[e];
          __asm__ volatile("" : "+v"(t));  // fp32, then one rounding to fp16 (as kernel (a))
          v[e] = (half_t)t;
        }
        *reinterpret_cast<half4*>(&st[br_st_off(lane & 31, c4)]) = v;
      }
    // The staging rows are private to the wave and a wave's LDS operations complete in
    // order; this only keeps the compiler from moving the reads above the writes.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // Staged chunk q of a channel: operand row j0 + q, k = i0 .. i0+7, i.e. lane
    // (j0 + q) % 32 + 32 (i0 / 8 % 2) of fragment tile (j0 / 32, i0 / 16).
    const size_t tile_h = ((size_t)(j0 >> 5) * p.kbn + (i0 >> 4)) * FragLayout::kTileHalfs +
                          (size_t)((j0 & 31) + 32 * ((i0 >> 3) & 1)) * 8;
    const rsrc_t ro = make_rsrc((is_b ? p.b : p.a) + ((size_t)bi * CL + ch_base) * plane_h + tile_h);
    const int q = lane & 7;
#pragma unroll
    for (int u = 0; u < CPW / 8; u++) {
      const int ch = 8 * u + (lane >> 3);
      bstore16(ro, (uint32_t)(ch * plane_h + q * 8) * 2u, ld16(&st[br_st_off(ch, q * 8)]));
    }
  };

  // Software pipeline as in kernel (a): the next tile's loads are in flight while this one
  // computes (ping-pong registers, unrolled by two, so no register copy waits on a load);
  // the first tile's loads go out before the weights.
  const int G = gridDim.x;
  TileLoads tA, tB;
  int tile = xcd_remap(blockIdx.x, G);
  load_tile(tile, tA);
  load_weights();
  for (; tile < p.ntiles; tile += 2 * G) {
    load_tile(tile + G, tB);
    process_tile(tile, tA);
    if (tile + G >= p.ntiles) break;
    load_tile(tile + 2 * G, tA);
    process_tile(tile + G, tB);
  }
}

hipError_t launch_bridge(const BridgeArgs& a, int grid, hipStream_t s) {
  if (a.mask)
    hipLaunchKernelGGL(tmu_bridge_kernel<true>, dim3(grid), dim3(NT), 0, s, a);
  else
    hipLaunchKernelGGL(tmu_bridge_kernel<false>, dim3(grid), dim3(NT), 0, s, a);
  return hipGetLastError();
}

}  // namespace esm
