// Kernel (b): the triangle contraction as an fp16 MFMA batched "A.B^T" GEMM,
//   x[n, i, j] = scale * sum_k a[n, i, k] * b[n, j, k],
// one channel n per grid z-slice, 128x128 output tiles, fp32 accumulation.
//
// Both operands are row-major with k contiguous (the incoming direction arrives
// pre-transposed from kernel (a)), so every MFMA fragment is one 16-byte LDS
// read. K advances in steps of 32 through a double-buffered LDS stage fed by
// 16-byte global loads into registers one step ahead; rows past L and columns
// past ld are zero-filled at load time, so no operand padding is read.
// Four waves in a 2x2 arrangement each own a 64x64 quadrant (2x2 MFMA 32x32x16
// tiles). The epilogue scales in fp32, rounds once to fp16 and stores through
// an LDS staging tile as 16-byte row segments.
#include "common.h"
#include "kernels.h"

namespace esm {

namespace {
constexpr int BM = kContractTile;  // rows (i) per tile
constexpr int BN = kContractTile;  // cols (j) per tile
constexpr int BK = 32;             // k per stage
constexpr int KS = BK + 8;         // LDS row stride (halfs) of an operand stage
constexpr int STAGE = (BM + BN) * KS;
constexpr int CS = BN + 8;         // LDS row stride (halfs) of the output staging tile
static_assert(BM * CS <= 2 * STAGE, "output staging must fit in the operand buffers");
}  // namespace

__global__ __launch_bounds__(256, 2) void tmu_contract_kernel(ContractArgs p) {
  __shared__ __align__(16) half_t smem[2 * STAGE];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 1, wn = wave & 1;
  const int tj = blockIdx.x, ti = blockIdx.y, n = blockIdx.z;
  const int L = p.L, ld = p.ld;
  const int i0 = ti * BM, j0 = tj * BN;
  const half_t* A = p.a + (size_t)n * L * ld;
  const half_t* B = p.b + (size_t)n * L * ld;

  // Loader: 4 x 16-byte chunks per thread per stage; u = 0,1 -> A rows, 2,3 -> B rows.
  half8 pre[4];
  auto gload = [&](int k0) {
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int id = tid + 256 * (u & 1);
      const int row = id >> 2, kc = id & 3;
      const int grow = (u < 2 ? i0 : j0) + row;
      const int k = k0 + kc * 8;
      const half_t* src = u < 2 ? A : B;
      pre[u] = (grow < L && k < ld) ? ld16(src + (size_t)grow * ld + k) : zero_half8();
    }
  };
  auto swrite = [&](int buf) {
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int id = tid + 256 * (u & 1);
      const int row = id >> 2, kc = id & 3;
      st16(smem + buf * STAGE + (u < 2 ? 0 : BM * KS) + row * KS + kc * 8, pre[u]);
    }
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int mi = 0; mi < 2; mi++)
#pragma unroll
    for (int ni = 0; ni < 2; ni++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[mi][ni][r] = 0.f;

  const int nk = (ld + BK - 1) / BK;
  gload(0);
  swrite(0);
  __syncthreads();
  for (int kt = 0; kt < nk; kt++) {
    const int buf = kt & 1;
    if (kt + 1 < nk) gload((kt + 1) * BK);
    const half_t* a_s = smem + buf * STAGE;
    const half_t* b_s = a_s + BM * KS;
#pragma unroll
    for (int kk = 0; kk < BK / 16; kk++) {
      half8 af[2], bf[2];
#pragma unroll
      for (int mi = 0; mi < 2; mi++)
        af[mi] = ld16(a_s + (wm * 64 + mi * 32 + (lane & 31)) * KS + kk * 16 + 8 * (lane >> 5));
#pragma unroll
      for (int ni = 0; ni < 2; ni++)
        bf[ni] = ld16(b_s + (wn * 64 + ni * 32 + (lane & 31)) * KS + kk * 16 + 8 * (lane >> 5));
#pragma unroll
      for (int mi = 0; mi < 2; mi++)
#pragma unroll
        for (int ni = 0; ni < 2; ni++) acc[mi][ni] = mfma32(af[mi], bf[ni], acc[mi][ni]);
    }
    if (kt + 1 < nk) swrite(buf ^ 1);
    __syncthreads();
  }

  // Epilogue: scale, round once, stage, 16-byte stores of whole row segments.
  half_t* c_s = smem;
#pragma unroll
  for (int mi = 0; mi < 2; mi++)
#pragma unroll
    for (int ni = 0; ni < 2; ni++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int row = wm * 64 + mi * 32 + acc_row32(r, lane);
        const int col = wn * 64 + ni * 32 + (lane & 31);
        c_s[row * CS + col] = (half_t)(acc[mi][ni][r] * p.scale);
      }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < (BM * BN / 8) / 256; u++) {
    const int id = tid + 256 * u;
    const int row = id >> 4, q = id & 15;
    const int gi = i0 + row, gj = j0 + q * 8;
    if (gi < L && gj < p.ldx) st16(p.x + ((size_t)n * L + gi) * p.ldx + gj, ld16(c_s + row * CS + q * 8));
  }
}

hipError_t launch_contract(const ContractArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(tmu_contract_kernel, dim3(a.tiles, a.tiles, a.batch), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace esm
