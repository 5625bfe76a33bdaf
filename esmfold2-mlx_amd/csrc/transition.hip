// Kernel (e): the pair transition, out = z + W3 act(W1 LN(z)) on every cell of the
// pair grid (cell-major [cells, C], C = 128), with act = ReLU (the block-stack
// workload's MLP) or SwiGLU, act = silu(W1 h) * (W2 h) (the reference's transition,
// fast_trunk.py:35-42, mlx_trunk.py:96-99). fp16 in/out, fp32 LayerNorm statistics and
// accumulation; the hidden activations are rounded once to fp16 for the second GEMM
// and the output once after the residual add (the reference's addmm residual,
// mlx_trunk_kernels.py:239).
//
// Persistent, one 4-wave workgroup per CU (one wave per SIMD, up to 512 registers):
// wave w owns hidden units [wU, wU + U) (U = H/4) and keeps its slices of W1 (and W2)
// and of W3 in registers for the whole launch (256 registers at H = 512), so the only
// per-tile traffic is z in and out and the partials through LDS. Per tile of
// 32 consecutive cells:
//   1. LayerNorm (16 lanes per cell) into an LDS tile n[cell][c]; the raw z stays in
//      registers for the residual;
//   2. first GEMM, transposed: D1[unit][cell] = W1[unit][:] . n[cell][:]
//      (v_mfma_f32_32x32x16_f16, A = W1 rows, B = n), one chain per 32-unit block;
//   3. act in fp32, rounded to fp16. A lane of D1 holds, for its cell, the units
//      {4h..4h+3, 8+4h..8+4h+3} (+16) of each 32-unit block (h = lane/32): exactly a
//      B fragment of the second GEMM if that GEMM's k order within a 16-unit step is
//      permuted the same way, so the activations go from accumulator to operand with
//      no data movement; W3's fragments are read in that order;
//   4. second GEMM: D2[ch][cell] = sum over the wave's units of W3[ch][unit] act[..],
//      a partial over U of the H units, one chain per 32-channel block;
//   5. the 4 partials meet in LDS (16-byte slots XOR-swizzled by the register quad, so
//      both the writes and the per-cell reads are free of bank conflicts), are summed in
//      wave order with z and leave as whole 256-byte cell rows.
// The next tile's z is loaded while this one computes.
#include "common.h"
#include "kernels.h"

namespace esm {

namespace {
constexpr int C = 128;          // pair channels
constexpr int TC = 32;          // cells per tile
constexpr int NWT = 4;          // waves per workgroup
constexpr int NTT = NWT * 64;   // threads
constexpr int NSTR = C + 8;     // LDS row stride (halfs) of the LayerNormed tile
constexpr int STAGE_ROWS = 256; // weight staging rows of 128 halfs (64 KB)
constexpr int RED_BYTES = NWT * 16 * 64 * 16;  // 4 waves x 16 quads x 64 lanes x 16 B = 64 KB
static_assert(STAGE_ROWS * C * 2 <= RED_BYTES, "weight staging fits the reduction area");
}  // namespace

template <int U, bool SWIGLU>
__global__ __launch_bounds__(NTT, 1) void transition_kernel(TransitionArgs p) {
  constexpr int UB = U / 32;      // 32-unit blocks per wave
  constexpr int H = NWT * U;      // hidden units
  static_assert(U == 64 || U == 128, "a wave's units lie in one 128-column piece of W3");
  __shared__ __align__(16) char smem[RED_BYTES + TC * NSTR * 2];
  half_t* stage = reinterpret_cast<half_t*>(smem);          // start-up: weight staging
  f32x4* red = reinterpret_cast<f32x4*>(smem);              // per tile: the 4 partials
  half_t* n_s = reinterpret_cast<half_t*>(smem + RED_BYTES);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 31, h = lane >> 5;
  const int u0 = wave * U;  // this wave's first unit

  // --- weights -> registers, through LDS with coalesced loads ------------------------------
  half8 wa1[UB][C / 16];                     // A fragments of W1 (and W2): row = unit, k = channel
  half8 wa2[SWIGLU ? UB : 1][C / 16];
  half8 wa3[C / 32][2 * UB];                 // A fragments of W3: row = channel, k = unit (permuted)
  auto rows_round = [&](const half_t* w, half8 (&dst)[UB][C / 16]) {
    // H rows of 128 halfs, 256 rows per round
    for (int r0 = 0; r0 < H; r0 += STAGE_ROWS) {
      RowStage<STAGE_ROWS, NTT> st;
      st.load(w + (size_t)r0 * C, tid);
      st.store(stage, tid);
      __syncthreads();
#pragma unroll
      for (int ub = 0; ub < UB; ub++) {
        const int row = u0 + 32 * ub + r - r0;  // wave-uniform range test below
        if (u0 + 32 * ub >= r0 && u0 + 32 * ub < r0 + STAGE_ROWS) {
#pragma unroll
          for (int ks = 0; ks < C / 16; ks++) dst[ub][ks] = staged_chunk(stage, row, 2 * ks + h);
        }
      }
      __syncthreads();
    }
  };
  rows_round(p.w1, wa1);
  if constexpr (SWIGLU) rows_round(p.w2, wa2);
  // W3 [C, H]: rounds of two 128-column pieces (128 rows each), staged as 256 rows.
  for (int c0 = 0; c0 < H; c0 += 256) {
    constexpr int PER = STAGE_ROWS * 16 / NTT;
    half8 v[PER];
#pragma unroll
    for (int i = 0; i < PER; i++) {
      const int q = tid + NTT * i, pc = q >> 11, ch = (q >> 4) & 127, j = q & 15;
      v[i] = (c0 + 128 * pc < H) ? ld16(p.w3 + (size_t)ch * H + c0 + 128 * pc + 8 * j) : zero_half8();
    }
#pragma unroll
    for (int i = 0; i < PER; i++) {
      const int q = tid + NTT * i, row = q >> 4, j = q & 15;
      st16(stage + row * 128 + 8 * (j ^ (row & 15)), v[i]);
    }
    __syncthreads();
    if (u0 >= c0 && u0 < c0 + 256) {
      const int piece_row0 = ((u0 - c0) >> 7) * 128;  // this wave's piece in the round
      const int col0 = u0 & 127;
#pragma unroll
      for (int ob = 0; ob < C / 32; ob++) {
        const int row = piece_row0 + 32 * ob + r;
#pragma unroll
        for (int j = 0; j < 2 * UB; j++) {
          // units 16j + {4h..4h+3} and 16j + 8 + {4h..4h+3}: two 8-byte halves of chunks
          const int ca = col0 + 16 * j + 4 * h, cb = ca + 8;
          const half_t* base = stage + row * 128;
          const half4 lo = *reinterpret_cast<const half4*>(base + 8 * ((ca >> 3) ^ (row & 15)) + (ca & 7));
          const half4 hi = *reinterpret_cast<const half4*>(base + 8 * ((cb >> 3) ^ (row & 15)) + (cb & 7));
          wa3[ob][j] = half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
      }
    }
    __syncthreads();
  }

  // LayerNorm parameters of this lane's 8 channels.
  const int ch0 = (lane & 15) * 8;
  float g[8], bb[8];
#pragma unroll
  for (int e = 0; e < 8; e++) {
    g[e] = p.ln_w[ch0 + e];
    bb[e] = p.ln_b[ch0 + e];
  }

  // Thread -> (cell tid/16 + 16 i, channels ch0 .. ch0+7) for the loads, the LayerNorm,
  // the residual and the stores. Cells past the end load zeros and store nothing.
  // The descriptors start at the tile's first cell, so the offsets stay small at any size
  // (a tile past the end, the pipeline's last prefetch, uses tile 0's and loads nothing).
  const size_t ncells = p.ncells;
  auto tile_base = [&](int tile) -> size_t { return (size_t)(tile < p.ntiles ? tile : 0) * TC * C; };
  auto cell_off = [&](int tile, int i) -> uint32_t {
    const int c = (tid >> 4) + 16 * i;
    return (size_t)tile * TC + c < ncells ? (uint32_t)(c * C + ch0) * 2u : kOOB;
  };
  auto load_tile = [&](int tile, half8 (&zq)[2]) {
    const rsrc_t rz = make_rsrc(p.z + tile_base(tile));
#pragma unroll
    for (int i = 0; i < 2; i++) zq[i] = bload16(rz, cell_off(tile, i));
  };

  const int G = gridDim.x;
  half8 zA[2], zB[2];
  int tile = blockIdx.x;
  load_tile(tile, zA);

  auto process = [&](int t, const half8 (&zq)[2]) {
    // 1. LayerNorm -> n_s
#pragma unroll
    for (int i = 0; i < 2; i++) st16(&n_s[((tid >> 4) + 16 * i) * NSTR + ch0], ln_row128_h(zq[i], g, bb, p.eps));
    __syncthreads();

    // 2. D1[unit][cell] (and the gate branch), one chain per unit block
    f32x16 d1[UB], d2[SWIGLU ? UB : 1];
#pragma unroll
    for (int ub = 0; ub < UB; ub++)
#pragma unroll
      for (int i = 0; i < 16; i++) {
        d1[ub][i] = 0.f;
        if constexpr (SWIGLU) d2[ub][i] = 0.f;
      }
#pragma unroll
    for (int ks = 0; ks < C / 16; ks++) {
      const half8 nb = ld16(&n_s[r * NSTR + 16 * ks + 8 * h]);
#pragma unroll
      for (int ub = 0; ub < UB; ub++) {
        d1[ub] = mfma32(wa1[ub][ks], nb, d1[ub]);
        if constexpr (SWIGLU) d2[ub] = mfma32(wa2[ub][ks], nb, d2[ub]);
      }
    }

    // 3. act -> fp16 B fragments of the second GEMM (registers 0-7 and 8-15 of a block)
    half8 act[2 * UB];
#pragma unroll
    for (int ub = 0; ub < UB; ub++)
#pragma unroll
      for (int i = 0; i < 16; i++) {
        float a = d1[ub][i];
        if constexpr (SWIGLU) {
          a = a * sigmoidf_fast(a) * d2[ub][i];
        } else {
          a = a > 0.f ? a : 0.f;
        }
        act[2 * ub + (i >> 3)][i & 7] = (half_t)a;
      }

    // 4. D2[ch][cell], partial over this wave's units
    f32x16 o2[C / 32];
#pragma unroll
    for (int ob = 0; ob < C / 32; ob++)
#pragma unroll
      for (int i = 0; i < 16; i++) o2[ob][i] = 0.f;
#pragma unroll
    for (int j = 0; j < 2 * UB; j++)
#pragma unroll
      for (int ob = 0; ob < C / 32; ob++) o2[ob] = mfma32(wa3[ob][j], act[j], o2[ob]);

    // 5. partials -> LDS: quad qd = 4 ob + r4 of lane l at slot l ^ qd
#pragma unroll
    for (int ob = 0; ob < C / 32; ob++)
#pragma unroll
      for (int r4 = 0; r4 < 4; r4++) {
        const int qd = 4 * ob + r4;
        red[(wave * 16 + qd) * 64 + (lane ^ qd)] =
            f32x4{o2[ob][4 * r4], o2[ob][4 * r4 + 1], o2[ob][4 * r4 + 2], o2[ob][4 * r4 + 3]};
      }
    __syncthreads();
    // thread (cell c, channels 8q .. 8q+7): quad q, rows 0-3 from lane c, 4-7 from lane 32+c
    const int q = lane & 15;
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int c = (tid >> 4) + 16 * i;
      f32x4 lo = red[q * 64 + (c ^ q)], hi = red[q * 64 + ((32 + c) ^ q)];
#pragma unroll
      for (int w = 1; w < NWT; w++) {
        lo += red[(w * 16 + q) * 64 + (c ^ q)];
        hi += red[(w * 16 + q) * 64 + ((32 + c) ^ q)];
      }
      half8 o;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        o[e] = (half_t)(lo[e] + (float)zq[i][e]);
        o[e + 4] = (half_t)(hi[e] + (float)zq[i][e + 4]);
      }
      bstore16(make_rsrc(p.out + tile_base(t)), cell_off(t, i), o);
    }
    __syncthreads();  // red and n_s are rewritten by the next tile
  };

  // Ping-pong register buffers for z, unrolled by two (no copy waits on a load).
  for (; tile < p.ntiles; tile += 2 * G) {
    load_tile(tile + G, zB);
    process(tile, zA);
    if (tile + G >= p.ntiles) break;
    load_tile(tile + 2 * G, zA);
    process(tile + G, zB);
  }
}

hipError_t launch_transition(const TransitionArgs& a, int grid, hipStream_t s) {
  const dim3 blk(NTT);
  if (a.w2 == nullptr && a.H == 512)
    ESM_LAUNCH((transition_kernel<128, false>), dim3(grid), blk, 0, s, a);
  else if (a.w2 == nullptr && a.H == 256)
    ESM_LAUNCH((transition_kernel<64, false>), dim3(grid), blk, 0, s, a);
  else if (a.w2 != nullptr && a.H == 256)
    ESM_LAUNCH((transition_kernel<64, true>), dim3(grid), blk, 0, s, a);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace esm
