// Kernel (b): the triangle contraction as an fp16 MFMA batched "A.B^T" GEMM,
//   x[n, i, j] = scale * sum_k a[n, i, k] * b[n, j, k],
// fp32 accumulation, one rounding to fp16.
//
// Both operands are row-major with k contiguous (the incoming direction arrives
// pre-transposed from kernel (a)), so every MFMA fragment is one 16-byte LDS read.
// A workgroup computes a 128 (i) x 256 (j) output block: for L <= 256 that is a
// whole row block of one channel, so each channel's B is requested by only
// ceil(L/128) workgroups and A exactly once. Four waves in a 2x2 arrangement
// each own 64x128 outputs (2x4 MFMA 32x32x16 tiles, 128 accumulators).
// K advances in steps of 32 through a double-buffered LDS stage fed by 16-byte
// global loads one step ahead; rows past L and columns past ld are zero-filled
// at load time.
//
// Workgroup order is XCD-aware: the dispatcher deals workgroup ids round-robin to
// the 8 XCDs, so ids are remapped so that consecutive logical blocks (the row
// blocks of one channel, which read the same B) run on the same XCD and share
// its L2.
#include "common.h"
#include "kernels.h"

namespace esm {

namespace {
constexpr int BM = 128;            // rows (i) per block
constexpr int BN = 256;            // cols (j) per block
constexpr int BK = 32;             // k per stage
constexpr int KS = BK + 8;         // LDS row stride (halfs) of an operand stage
constexpr int STAGE = (BM + BN) * KS;
constexpr int CS = BN + 8;         // LDS row stride (halfs) of the output staging tile
constexpr int SMEM = (2 * STAGE > BM * CS) ? 2 * STAGE : BM * CS;
constexpr int CHUNKS = (BM + BN) * BK / 8 / 256;  // 16-byte loads per thread per stage
static_assert((BM + BN) * BK / 8 % 256 == 0, "stage must split evenly over 256 threads");
static_assert(BM * 4 % 256 == 0, "A chunks must fill whole loader passes");
}  // namespace

__global__ __launch_bounds__(256, 2) void tmu_contract_kernel(ContractArgs p) {
  __shared__ __align__(16) half_t smem[SMEM];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int L = p.L, ld = p.ld;

  // XCD-aware remap of the workgroup id to a logical block index (a bijection).
  const int t = xcd_remap(blockIdx.x, gridDim.x);
  const int nrb = (L + BM - 1) / BM, ncb = (L + BN - 1) / BN;
  const int rb = t % nrb;
  const int cb = (t / nrb) % ncb;
  const int ch = t / (nrb * ncb);
  const int i0 = rb * BM, j0 = cb * BN;
  // Operand rows i0.. of A and j0.. of B; lanes past L or ld, and the prefetch past the
  // last stage, use an out-of-range offset: zeros, no memory traffic, no branch.
  const rsrc_t rA = make_rsrc(p.a + ((size_t)ch * L + i0) * ld);
  const rsrc_t rB = make_rsrc(p.b + ((size_t)ch * L + j0) * ld);
  const int nk = (ld + BK - 1) / BK;

  half8 pre[CHUNKS];
  auto gload = [&](int kt) {
#pragma unroll
    for (int u = 0; u < CHUNKS; u++) {
      const int id = tid + 256 * u;
      const bool isA = u < BM * 4 / 256;  // a compile-time split: chunks 0..BM*4-1 are A rows
      const int r = isA ? id >> 2 : (id - BM * 4) >> 2;
      const int k = kt * BK + (id & 3) * 8;
      const bool ok = kt < nk && (isA ? i0 : j0) + r < L && k < ld;
      pre[u] = bload16(isA ? rA : rB, ok ? (uint32_t)(r * ld + k) * 2u : kOOB);
    }
  };
  auto swrite = [&](int buf) {
#pragma unroll
    for (int u = 0; u < CHUNKS; u++) {
      const int id = tid + 256 * u;
      const int kc = id & 3;
      const int row = id >> 2;  // A rows 0..BM-1, then B rows follow them in the stage
      st16(smem + buf * STAGE + row * KS + kc * 8, pre[u]);
    }
  };

  f32x16 acc[2][4];
#pragma unroll
  for (int mi = 0; mi < 2; mi++)
#pragma unroll
    for (int ni = 0; ni < 4; ni++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[mi][ni][r] = 0.f;

  gload(0);
  swrite(0);
  __syncthreads();
  for (int kt = 0; kt < nk; kt++) {
    const int buf = kt & 1;
    gload(kt + 1);  // unconditional: past the last stage it reads nothing
    const half_t* a_s = smem + buf * STAGE;
    const half_t* b_s = a_s + BM * KS;
#pragma unroll
    for (int kk = 0; kk < BK / 16; kk++) {
      half8 af[2], bf[4];
#pragma unroll
      for (int mi = 0; mi < 2; mi++)
        af[mi] = ld16(a_s + (wm * 64 + mi * 32 + (lane & 31)) * KS + kk * 16 + 8 * (lane >> 5));
#pragma unroll
      for (int ni = 0; ni < 4; ni++)
        bf[ni] = ld16(b_s + (wn * 128 + ni * 32 + (lane & 31)) * KS + kk * 16 + 8 * (lane >> 5));
#pragma unroll
      for (int mi = 0; mi < 2; mi++)
#pragma unroll
        for (int ni = 0; ni < 4; ni++) acc[mi][ni] = mfma32(af[mi], bf[ni], acc[mi][ni]);
    }
    swrite(buf ^ 1);
    __syncthreads();
  }

  // Epilogue: scale, round once, stage, 16-byte stores of whole row segments.
  half_t* c_s = smem;
#pragma unroll
  for (int mi = 0; mi < 2; mi++)
#pragma unroll
    for (int ni = 0; ni < 4; ni++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int row = wm * 64 + mi * 32 + acc_row32(r, lane);
        const int col = wn * 128 + ni * 32 + (lane & 31);
        c_s[row * CS + col] = (half_t)(acc[mi][ni][r] * p.scale);
      }
  __syncthreads();
  const rsrc_t rX = make_rsrc(p.x + ((size_t)ch * L + i0) * p.ldx + j0);
#pragma unroll
  for (int u = 0; u < (BM * BN / 8) / 256; u++) {
    const int id = tid + 256 * u;
    const int row = id / (BN / 8), q = id % (BN / 8);
    const bool ok = i0 + row < L && j0 + q * 8 < p.ldx;
    bstore16(rX, ok ? (uint32_t)(row * p.ldx + q * 8) * 2u : kOOB, ld16(c_s + row * CS + q * 8));
  }
}

hipError_t launch_contract(const ContractArgs& a, hipStream_t s) {
  const long long blocks = (long long)a.batch * ((a.L + BM - 1) / BM) * ((a.L + BN - 1) / BN);
  hipLaunchKernelGGL(tmu_contract_kernel, dim3((unsigned)blocks), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace esm
