// Kernel (a): input LayerNorm -> C->4c projection (MFMA) -> sigmoid gates ->
// pair mask -> channel-major operands a, b.
//
// Persistent, one 8-wave workgroup per CU (2 waves per SIMD), walking tiles of 64
// cells along one "line" of the pair grid: cells (line, pos0..pos0+63) for the
// outgoing layout, cells (pos0..pos0+63, line) for the transposed (incoming) layout.
// Each cell's C channels are one contiguous 256-byte read.
//
// Waves 0-3 own channels [32w, 32w+32) of a, waves 4-7 the same channels of b; each
// keeps its slice of proj_bundle.weight (signal and gate rows of those channels) in
// VGPRs as MFMA B-fragments for the whole launch, read once through LDS with coalesced
// loads. The projection runs as
//   D[cell][channel] = LN(z)[cell][:] . W[channel][:]   (v_mfma_f32_32x32x16_f16)
// with the two 32-cell halves of a tile interleaved, so 4 independent accumulator
// chains keep the MFMA pipe full (the 16x16x32 form needs ~16 chains for the same
// rate). Each lane ends with groups of 4 consecutive cells of one channel for the
// signal and the gate alike:
// the gate is applied in fp32 straight from the accumulators and rounded once to
// fp16 (as the reference's gate_cf, mlx_trunk_kernels.py:60-64). The results are
// staged per wave in LDS and leave as whole 128-byte row segments (8 lanes x 16 B
// per channel row): scattered 32-byte pieces of rows measured 2x slower.
//
// Per tile: MFMA + gate + staging + store from a double-buffered LDS tile of LayerNormed
// cells, then one barrier. The LayerNorm (16 lanes per cell, v_dot2_f32_f16 statistics) of
// the next tile is done by the a-waves alone after their stores: each SIMD's a-wave finishes
// its products and gate well before the b-wave that shares the SIMD, and a lone wave leaves
// most of the SIMD's VALU issue slots free, so the normalisation runs under the b-wave's
// gate instead of in a phase of its own (17.2 -> 16.6 us). The z of the tile after next is
// loaded while this one computes. Every global access is an unconditional buffer
// instruction (out-of-range lanes use an offset the hardware drops), so the
// compiler's wait counts stay exact and the prefetch stays in flight.
#include "common.h"
#include "kernels.h"

namespace esm {

namespace {
constexpr int C = 128;                 // pair channels
constexpr int CL = 128;                // latent channels
constexpr int TM = kCellTile;          // cells per tile
constexpr int NS = C + 8;              // LDS row stride (halfs) of the normalised tile
constexpr int NW = 8;                  // waves per workgroup
constexpr int CPW = 2 * CL / NW;       // channels per wave (of a for waves 0-3, of b for 4-7)
constexpr int CPT = TM * 16 / (NW / 2 * 64);  // cells LayerNormed per a-wave thread per tile
static_assert(CPW == 32, "one 32-column MFMA tile of channels per wave");
static_assert(TM == 64, "a staged output row is 64 cells = 128 bytes = 8 chunks");
}  // namespace

// Output staging: per wave, 32 channel rows of 64 cells (128 bytes, 8 chunks of 16 B),
// chunk q of row ch stored at physical chunk q ^ ((ch >> 1) & 7). The 8-byte writes of
// one accumulator group (32 rows, 2 lanes each) take the minimum two passes and the
// 16-byte reads of two whole rows cover all 64 banks once.
DEV int st_off(int ch, int cell) {  // in halfs
  return ch * TM + 8 * ((cell >> 3) ^ ((ch >> 1) & 7)) + (cell & 7);
}

template <bool HAS_MASK, bool FRAG>
__global__ __launch_bounds__(NW * 64, 1) void tmu_project_kernel(ProjectArgs p) {
  __shared__ __align__(16) half_t n_s[2][TM * NS];
  __shared__ __align__(16) float m_s[2][TM];
  __shared__ __align__(16) half_t st_s[NW][CPW * TM];
  __shared__ __align__(16) half_t w_s[2 * CL * C];  // weight staging, start-up only

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: keeps descriptors scalar
  const int L = p.L;
  constexpr bool has_mask = HAS_MASK;

  // Weight B-fragments: column = channel, k = 16 ks + 8 (lane/32) + e. Rows of
  // proj_bundle.weight: signal s_a = [0, c), s_b = [c, 2c); gate g_a = [2c, 3c), g_b = [3c, 4c).
  const int is_b = wave >= NW / 2;
  const int ch_base = CPW * (wave - is_b * (NW / 2));  // first channel of this wave (of a or b)
  // The bundle streams through LDS in two coalesced rounds of 256 rows: the signal rows
  // [0, 2c), then the gate rows [2c, 4c); both rounds' loads are in flight together.
  half8 ws[C / 16], wg[C / 16];
  auto load_weights = [&] {
    RowStage<2 * CL, NW * 64> r0, r1;
    r0.load(p.w, tid);
    r1.load(p.w + 2 * CL * C, tid);
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
  };
  // LayerNorm parameters of this lane's 8 channels.
  const int ch0 = (lane & 15) * 8;
  float g[8], bb[8];
#pragma unroll
  for (int e = 0; e < 8; e++) {
    g[e] = p.ln_w[ch0 + e];
    bb[e] = p.ln_b[ch0 + e];
  }

  // Tile coordinates. Row-major planes: `line` is the fixed grid index, positions
  // pos0 .. pos0+63 vary. FRAG: a block of 8 x 8 cells, operand rows line .. line+7 and
  // k pos0 .. pos0+7 (tile cell cl = 8 dr + dc is row line + dr, k pos0 + dc).
  auto coords = [&](int tile, int& bi, int& line, int& pos0) {
    if constexpr (FRAG) {
      const int per = p.tiles_per_line * p.tiles_per_line;
      bi = tile / per;
      const int t = tile - bi * per;
      const int tr = t / p.tiles_per_line;
      line = 8 * tr;
      pos0 = 8 * (t - tr * p.tiles_per_line);
    } else {
      const int bl = tile / p.tiles_per_line;
      pos0 = (tile - bl * p.tiles_per_line) * TM;
      bi = bl / L;
      line = bl - bi * L;
    }
  };
  const uint32_t cstride = p.transpose ? (uint32_t)L : 1u;  // cell stride along the tile
  // Offset (in cells, from the tile's first cell) of tile cell cl, and whether it is in range.
  auto cell_off = [&](int cl) -> uint32_t {
    if constexpr (FRAG) {
      const uint32_t dr = cl >> 3, dc = cl & 7;   // operand row line + dr, k pos0 + dc
      return p.transpose ? dc * (uint32_t)L + dr : dr * (uint32_t)L + dc;
    } else {
      return cl * cstride;
    }
  };
  auto cell_ok = [&](int line, int pos0, int cl) -> bool {
    if constexpr (FRAG) return line + (cl >> 3) < L && pos0 + (cl & 7) < L;
    else return pos0 + cl < L;
  };

  // Issue one tile's loads (the a-waves, threads 0 .. 255): z (16 lanes per cell, 8 channels
  // per lane) and the raw mask. A tile index past the end (the pipeline's last prefetch) loads
  // nothing.
  auto load_tile = [&](int tile, half8 (&zq)[CPT], uint16_t (&mq)[CPT]) {
    const bool live = tile < p.ntiles;
    int bi, line, pos0;
    coords(live ? tile : 0, bi, line, pos0);
    const size_t cb = (size_t)bi * L * L + (p.transpose ? (size_t)pos0 * L + line : (size_t)line * L + pos0);
    // (FRAG: the tile's first cell is operand row `line`, k `pos0`: cell (line, pos0), or
    // (pos0, line) transposed, the same formula)
    const rsrc_t rz = make_rsrc(p.z + cb * C);
    const rsrc_t rm = make_rsrc(has_mask ? (const void*)(p.mask + cb) : (const void*)p.z);
    (void)rm;
#pragma unroll
    for (int it = 0; it < CPT; it++) {
      const int cl = (tid >> 4) + (NW * 2) * it;
      const bool ok = live && cell_ok(line, pos0, cl);
      zq[it] = bload16(rz, ok ? (uint32_t)(cell_off(cl) * C + ch0) * 2u : kOOB);
      if (has_mask) mq[it] = bload2(rm, ok ? cell_off(cl) * 2u : kOOB);
    }
  };

  // LayerNorm of a tile -> LDS buffer nb, by the a-waves only (each SIMD's a-wave finishes its
  // products and gate before its b-wave, and normalises the next tile while the b-wave still
  // gates this one). Double-buffered: the b-waves may still read the other buffer.
  auto ln_tile = [&](int tile, const half8 (&zq)[CPT], const uint16_t (&mq)[CPT], int nb) {
    int bi, line, pos0;
    coords(tile, bi, line, pos0);
    half_t* ns = n_s[nb];
#pragma unroll
    for (int it = 0; it < CPT; it++) {
      const int cl = (tid >> 4) + (NW * 2) * it;
      half8 o = ln_row128_h(zq[it], g, bb, p.eps);
      // Cells past L (zeros from the range-checked loads) enter the projection as zeros,
      // so their padded outputs [L, ld) are exactly 0 with or without a mask (their
      // LayerNorm would be 0 * rsqrt(eps), NaN for eps = 0).
      const bool cell_in = cell_ok(line, pos0, cl);
      if (!cell_in) o = zero_half8();
      st16(&ns[cl * NS + ch0], o);
      if (has_mask && (lane & 15) == 0) m_s[nb][cl] = cell_in ? h2f(mq[it]) : 0.f;
    }
  };

  auto process_tile = [&](int tile, int nb) {
    int bi, line, pos0;
    coords(tile, bi, line, pos0);
    half_t* ns = n_s[nb];
    // Projection of both 32-cell halves (4 accumulator chains), gate in fp32, groups of
    //    4 cells of one channel per lane staged (8 bytes) in this wave's LDS rows.
    half_t* st = st_s[wave];
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
        const half8 af = ld16(&ns[(32 * h + (lane & 31)) * NS + 16 * ks + 8 * (lane >> 5)]);
        as[h] = mfma32(af, ws[ks], as[h]);
        ag[h] = mfma32(af, wg[ks], ag[h]);
      }
    }
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
      for (int r4 = 0; r4 < 4; r4++) {
        const int c4 = 32 * h + acc_row32(4 * r4, lane);  // first of this group's 4 cells
        // (a padding cell's signal is already 0: zero LayerNorm row)
        const f32x4 m4 = has_mask ? *reinterpret_cast<const f32x4*>(&m_s[nb][c4]) : f32x4{1.f, 1.f, 1.f, 1.f};
        half4 v;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          float t = as[h][4 * r4 + e] * sigmoidf_fast(ag[h][4 * r4 + e]);
          if (has_mask) t *= m4[e];
          // fp32 materialised, then one rounding to fp16: otherwise the compiler may fold the
          // last multiply and the conversion into one mixed-precision FMA in one inlined copy
          // and not in another, and the same value would round differently by position
          __asm__ volatile("" : "+v"(t));
          v[e] = (half_t)t;
        }
        *reinterpret_cast<half4*>(&st[st_off(lane & 31, c4)]) = v;
      }
    // The staging rows are private to the wave and a wave's LDS operations complete in
    // order; this only keeps the compiler from moving the reads above the writes.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // 3. Whole 128-byte row segments: 8 lanes x 16 B per channel row, 8 rows per store.
    //    Chunks at or past ld are dropped by the buffer range check. FRAG: the staged row
    //    of a channel (8 operand rows x 8 k) is lanes 32 (pos0 / 8 % 2) + line % 32 .. +7
    //    of one fragment tile: again one whole 128-byte segment.
    const int q = lane & 7;
    if constexpr (FRAG) {
      const size_t tile_h = ((size_t)(line >> 5) * p.kbn + (pos0 >> 4)) * FragLayout::kTileHalfs +
                            (size_t)((line & 31) + 32 * ((pos0 >> 3) & 1)) * 8;
      const size_t plane_h = (size_t)p.rbn * p.kbn * FragLayout::kTileHalfs;
      const rsrc_t ro = make_rsrc((is_b ? p.b : p.a) + ((size_t)bi * CL + ch_base) * plane_h + tile_h);
#pragma unroll
      for (int u = 0; u < CPW / 8; u++) {
        const int ch = 8 * u + (lane >> 3);
        bstore16(ro, (uint32_t)(ch * plane_h + q * 8) * 2u, ld16(&st[st_off(ch, q * 8)]));
      }
    } else {
      const size_t row0 = ((size_t)bi * CL + ch_base) * L + line;  // this wave's first channel row
      const rsrc_t ro = make_rsrc((is_b ? p.b : p.a) + row0 * p.ld + pos0);
      const bool okq = pos0 + q * 8 < p.ld;
#pragma unroll
      for (int u = 0; u < CPW / 8; u++) {
        const int ch = 8 * u + (lane >> 3);
        const uint32_t off = okq ? (uint32_t)((size_t)ch * L * p.ld + q * 8) * 2u : kOOB;
        bstore16(ro, off, ld16(&st[st_off(ch, q * 8)]));
      }
    }
  };

  // Software pipeline: the a-waves keep the next-but-one tile's loads in flight while this
  // tile computes and normalise the next tile after their stores (ping-pong register buffers,
  // unrolled by two so no register copy waits on a load; the loads of a tile are issued before
  // the stores that precede its LayerNorm, so waiting for them never waits for the stores).
  // Start-up order: the first tile's z goes out before the 16 KB of weights per wave.
  const int G = gridDim.x;
  half8 zA[CPT], zB[CPT];
  uint16_t mA[CPT] = {}, mB[CPT] = {};
  int tile = blockIdx.x;
  if (!is_b) load_tile(tile, zA, mA);
  load_weights();
  if (!is_b) {
    ln_tile(tile, zA, mA, 0);
    load_tile(tile + G, zB, mB);
  }
  __syncthreads();  // tile 0 normalised
  // One barrier per tile: it publishes the next tile's normalised rows and retires this
  // tile's reads of the buffer the a-waves write next.
  for (; tile < p.ntiles; tile += 2 * G) {
    process_tile(tile, 0);
    if (!is_b) {
      if (tile + G < p.ntiles) ln_tile(tile + G, zB, mB, 1);
      load_tile(tile + 2 * G, zA, mA);
    }
    __syncthreads();
    if (tile + G >= p.ntiles) break;
    process_tile(tile + G, 1);
    if (!is_b) {
      if (tile + 2 * G < p.ntiles) ln_tile(tile + 2 * G, zA, mA, 0);
      load_tile(tile + 3 * G, zB, mB);
    }
    __syncthreads();
  }
}

hipError_t launch_project(const ProjectArgs& a, int grid, hipStream_t s) {
  if (a.frag) {
    if (a.mask)
      ESM_LAUNCH((tmu_project_kernel<true, true>), dim3(grid), dim3(NW * 64), 0, s, a);
    else
      ESM_LAUNCH((tmu_project_kernel<false, true>), dim3(grid), dim3(NW * 64), 0, s, a);
  } else {
    if (a.mask)
      ESM_LAUNCH((tmu_project_kernel<true, false>), dim3(grid), dim3(NW * 64), 0, s, a);
    else
      ESM_LAUNCH((tmu_project_kernel<false, false>), dim3(grid), dim3(NW * 64), 0, s, a);
  }
  return hipGetLastError();
}

}  // namespace esm
