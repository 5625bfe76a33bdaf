// Kernel (a): input LayerNorm -> C->4c projection (MFMA) -> sigmoid gates ->
// pair mask -> channel-major operands a, b.
//
// Persistent: each workgroup keeps its share of proj_bundle.weight in VGPRs for
// the whole launch and walks cell tiles with a grid stride. A tile is 64 cells
// along one "line" of the pair grid: cells (line, pos0..pos0+63) for the
// outgoing layout, cells (pos0..pos0+63, line) for the transposed (incoming)
// layout. Either way each cell's C channels are one contiguous 256-byte read and
// each output row segment (one channel, 64 positions) is one contiguous 128-byte
// write, staged through LDS so every global access is a 16-byte vector.
//
// Wave w of the 4 computes channels [32w, 32w+32) of both a and b:
//   acc[0] = s_a rows, acc[1] = g_a rows, acc[2] = s_b rows, acc[3] = g_b rows
// so the signal and gate of one (channel, cell) land in the same lane and
// register: the gate is applied in fp32 straight from the accumulators and
// rounded once to fp16 (as the reference's gate_cf, mlx_trunk_kernels.py:60-64).
#include "common.h"
#include "kernels.h"

namespace esm {

namespace {
constexpr int C = 128;                 // pair channels
constexpr int CL = 128;                // latent channels
constexpr int TM = kCellTile;          // cells per tile
constexpr int NS = C + 8;              // LDS row stride (halfs) of the normalised tile
constexpr int SS = TM + 8;             // LDS row stride (halfs) of the output staging rows
}  // namespace

__global__ __launch_bounds__(256, 1) void tmu_project_kernel(ProjectArgs p) {
  __shared__ __align__(16) half_t n_s[TM * NS];
  __shared__ __align__(16) half_t st_s[4][2][32 * SS];
  __shared__ float m_s[TM];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int L = p.L;

  // This wave's weight rows as MFMA A-fragments: rt = 0 s_a, 1 g_a, 2 s_b, 3 g_b.
  half8 wr[4][C / 16];
  {
    const int base[4] = {0, 2 * CL, CL, 3 * CL};
    const int row = 32 * wave + (lane & 31);
#pragma unroll
    for (int rt = 0; rt < 4; rt++)
#pragma unroll
      for (int ks = 0; ks < C / 16; ks++)
        wr[rt][ks] = ld16(p.w + (size_t)(base[rt] + row) * C + ks * 16 + 8 * (lane >> 5));
  }
  // LayerNorm parameters of this lane's 8 channels.
  const int ch0 = (lane & 15) * 8;
  float g[8], bb[8];
#pragma unroll
  for (int e = 0; e < 8; e++) {
    g[e] = p.ln_w[ch0 + e];
    bb[e] = p.ln_b[ch0 + e];
  }

  for (int tile = blockIdx.x; tile < p.ntiles; tile += gridDim.x) {
    const int bl = tile / p.tiles_per_line;
    const int pos0 = (tile - bl * p.tiles_per_line) * TM;
    const int bi = bl / L, line = bl - bi * L;
    const size_t plane = (size_t)bi * L * L;

    // 1. Load 64 cells (16 lanes per cell, 8 channels per lane), LayerNorm, -> LDS.
#pragma unroll
    for (int it = 0; it < 4; it++) {
      const int cl = (tid >> 4) + 16 * it;
      const int pos = pos0 + cl;
      half8 h = zero_half8();
      float mval = 0.f;  // cells past L get a zero mask so their padded outputs are exactly 0
      if (pos < L) {
        const size_t cell = plane + (p.transpose ? (size_t)pos * L + line : (size_t)line * L + pos);
        h = ld16(p.z + cell * C + ch0);
        mval = p.mask ? (float)p.mask[cell] : 1.f;
      }
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; e++) v[e] = (float)h[e];
      ln_row128(v, g, bb, p.eps);
      half8 o;
#pragma unroll
      for (int e = 0; e < 8; e++) o[e] = (half_t)v[e];
      st16(&n_s[cl * NS + ch0], o);
      if ((lane & 15) == 0) m_s[cl] = mval;
    }
    __syncthreads();

    // 2. Projection on MFMA, gate in fp32, stage fp16 channel rows in LDS.
#pragma unroll
    for (int cs = 0; cs < TM / 32; cs++) {
      f32x16 acc[4];
#pragma unroll
      for (int rt = 0; rt < 4; rt++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[rt][r] = 0.f;
#pragma unroll
      for (int ks = 0; ks < C / 16; ks++) {
        const half8 bf = ld16(&n_s[(cs * 32 + (lane & 31)) * NS + ks * 16 + 8 * (lane >> 5)]);
#pragma unroll
        for (int rt = 0; rt < 4; rt++) acc[rt] = mfma32(wr[rt][ks], bf, acc[rt]);
      }
      const int cl = cs * 32 + (lane & 31);
      const float mval = m_s[cl];
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int ch = acc_row32(r, lane);
        st_s[wave][0][ch * SS + cl] = (half_t)(acc[0][r] * sigmoidf_fast(acc[1][r]) * mval);
        st_s[wave][1][ch * SS + cl] = (half_t)(acc[2][r] * sigmoidf_fast(acc[3][r]) * mval);
      }
    }
    __syncthreads();

    // 3. Store this wave's 32 channel rows of a and b: 8 lanes x 16 B per row.
#pragma unroll
    for (int u = 0; u < 8; u++) {
      const int which = u >> 2;
      const int ch = (u & 3) * 8 + (lane >> 3);
      const int q = lane & 7;
      const int pos = pos0 + q * 8;
      if (pos < p.ld) {
        const half8 v = ld16(&st_s[wave][which][ch * SS + q * 8]);
        half_t* dst = (which ? p.b : p.a) + (((size_t)bi * CL + 32 * wave + ch) * L + line) * p.ld + pos;
        st16(dst, v);
      }
    }
  }
}

hipError_t launch_project(const ProjectArgs& a, int grid, hipStream_t s) {
  hipLaunchKernelGGL(tmu_project_kernel, dim3(grid), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace esm
