// Kernel (b): the triangle contraction as an fp16 MFMA batched "A.B^T" GEMM,
//   x[n, i, j] = scale * sum_k a[n, i, k] * b[n, j, k],
// fp32 accumulation, one rounding to fp16.
//
// Both operands are row-major with k contiguous (the incoming direction arrives
// pre-transposed from kernel (a)), so every MFMA fragment is one 16-byte LDS read.
// A workgroup computes a 128 (i) x 128 (j) output block; four waves in a 2x2
// arrangement each own 64x64 outputs (2x2 MFMA 32x32x16 tiles, 64 accumulators).
// Two workgroups share a CU (73.7 KB of LDS each), so one's operand stream overlaps
// the other's start-up and output stores: with a single workgroup per CU those
// phases ran back to back and took ~40% of the kernel.
//
// The kernel is bound by how fast one CU can pull operands through its L1 miss path,
// so the pipeline keeps two 32 KB stages in flight per workgroup: K advances in steps
// of 64 (each operand row contributes one whole 128-byte line per stage), stage kt+2
// is requested into registers while stage kt is multiplied out of LDS and stage kt+1
// (already in registers) is written to the other LDS buffer. Rows past L and columns
// past ld are zero-filled at load time.
//
// Each MFMA computes the transposed tile (B rows as the "A" operand), so every lane
// ends with 4 consecutive j of one i: the result is staged with 8-byte LDS writes and
// leaves as whole 16-byte row chunks.
//
// Workgroup order is XCD-aware: the dispatcher deals workgroup ids round-robin to
// the 8 XCDs, so ids are remapped so that consecutive logical blocks (the blocks of
// one channel, which read the same A rows and B rows) run on the same XCD and share
// its L2.
#include "common.h"
#include "kernels.h"

namespace esm {

namespace {
constexpr int BM = 128;            // rows (i) per block
constexpr int BN = 128;            // cols (j) per block
constexpr int BK = 64;             // k per stage: one 128-byte line per operand row
constexpr int KC = BK / 8;         // 16-byte chunks per row per stage
constexpr int KS = BK + 8;         // LDS row stride (halfs): 36 dwords, 16 consecutive rows
                                   // start in 16 distinct 4-bank groups
constexpr int STAGE = (BM + BN) * KS;
constexpr int CS = BN + 8;         // LDS row stride (halfs) of the output staging tile
constexpr int SMEM = (2 * STAGE > BM * CS) ? 2 * STAGE : BM * CS;
constexpr int NT = 256;            // threads per workgroup
constexpr int CHUNKS = (BM + BN) * KC / NT;  // 16-byte loads per thread per stage
constexpr int ACHUNKS = BM * KC / NT;        // of which A rows
static_assert((BM + BN) * KC % NT == 0 && BM * KC % NT == 0, "stage must split evenly over the threads");
static_assert(2 * SMEM * 2 <= 160 * 1024, "LDS budget: two workgroups per CU");
}  // namespace

__global__ __launch_bounds__(NT, 2) void tmu_contract_kernel(ContractArgs p) {
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
  // Operand rows i0.. of A and j0.. of B; lanes past L or ld, and the prefetches past
  // the last stage, use an out-of-range offset: zeros, no memory traffic, no branch.
  const rsrc_t rA = make_rsrc(p.a + ((size_t)ch * L + i0) * ld);
  const rsrc_t rB = make_rsrc(p.b + ((size_t)ch * L + j0) * ld);
  const int nk = (ld + BK - 1) / BK;

  auto gload = [&](half8 (&pre)[CHUNKS], int kt) {
#pragma unroll
    for (int u = 0; u < CHUNKS; u++) {
      const int id = tid + NT * u;
      const bool isA = u < ACHUNKS;  // compile-time split: A rows first, then B rows
      const int r = isA ? id / KC : (id - BM * KC) / KC;
      const int k = kt * BK + (id % KC) * 8;
      const bool ok = (isA ? i0 : j0) + r < L && k < ld;  // k >= ld past the last stage
      pre[u] = bload16(isA ? rA : rB, ok ? (uint32_t)(r * ld + k) * 2u : kOOB);
    }
  };
  auto swrite = [&](const half8 (&pre)[CHUNKS], int buf) {
#pragma unroll
    for (int u = 0; u < CHUNKS; u++) {
      const int id = tid + NT * u;
      const int row = id / KC;  // A rows 0..BM-1, then the B rows follow them in the stage
      st16(smem + buf * STAGE + row * KS + (id % KC) * 8, pre[u]);
    }
  };

  constexpr int NI = BN / 64;  // 32-column tiles per wave
  f32x16 acc[2][NI];
#pragma unroll
  for (int mi = 0; mi < 2; mi++)
#pragma unroll
    for (int ni = 0; ni < NI; ni++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[mi][ni][r] = 0.f;

  auto compute = [&](int buf) {
    const half_t* a_s = smem + buf * STAGE;
    const half_t* b_s = a_s + BM * KS;
#pragma unroll
    for (int kk = 0; kk < BK / 16; kk++) {
      half8 af[2], bf[NI];
#pragma unroll
      for (int mi = 0; mi < 2; mi++)
        af[mi] = ld16(a_s + (wm * 64 + mi * 32 + (lane & 31)) * KS + kk * 16 + 8 * (lane >> 5));
#pragma unroll
      for (int ni = 0; ni < NI; ni++)
        bf[ni] = ld16(b_s + (wn * (BN / 2) + ni * 32 + (lane & 31)) * KS + kk * 16 + 8 * (lane >> 5));
#pragma unroll
      for (int mi = 0; mi < 2; mi++)
#pragma unroll
        for (int ni = 0; ni < NI; ni++) acc[mi][ni] = mfma32(bf[ni], af[mi], acc[mi][ni]);
    }
  };

  // Two register stages: while stage kt is multiplied, stage kt+1 sits in one register
  // set (then goes to the other LDS buffer, last read in stage kt-1, before the barrier
  // that ends this step) and stage kt+2 loads into the other set. Unrolled by two so
  // the register sets are static; a step past the last stage multiplies zeros.
  half8 r0[CHUNKS], r1[CHUNKS];
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

  // Epilogue: scale, round once, stage, 16-byte stores of whole row segments. Lane l
  // holds, per tile and register group g, x[i = l % 32][j = 8g + 4(l / 32) .. +3].
  half_t* c_s = smem;
#pragma unroll
  for (int mi = 0; mi < 2; mi++)
#pragma unroll
    for (int ni = 0; ni < NI; ni++)
#pragma unroll
      for (int g4 = 0; g4 < 4; g4++) {
        const int row = wm * 64 + mi * 32 + (lane & 31);
        const int col = wn * (BN / 2) + ni * 32 + acc_row32(4 * g4, lane);
        half4 v;
#pragma unroll
        for (int e = 0; e < 4; e++) v[e] = (half_t)(acc[mi][ni][4 * g4 + e] * p.scale);
        *reinterpret_cast<half4*>(c_s + row * CS + col) = v;
      }
  __syncthreads();
  const rsrc_t rX = make_rsrc(p.x + ((size_t)ch * L + i0) * p.ldx + j0);
#pragma unroll
  for (int u = 0; u < (BM * BN / 8) / NT; u++) {
    const int id = tid + NT * u;
    const int row = id / (BN / 8), q = id % (BN / 8);
    const bool ok = i0 + row < L && j0 + q * 8 < p.ldx;
    bstore16(rX, ok ? (uint32_t)(row * p.ldx + q * 8) * 2u : kOOB, ld16(c_s + row * CS + q * 8));
  }
}

// The same contraction on operands in FragLayout (written so by kernel (a) in the fused
// forward): every MFMA fragment is one fully coalesced 1 KB load straight into registers,
// so there is no LDS staging and no barrier in the K loop. A workgroup computes a 128 x 128
// block as 2 x 2 waves of 64 x 64 (the two waves that share A rows, or B rows, read them
// within a few cycles of each other: one L2 fetch); each wave keeps NSF k-steps of
// fragments in flight. Lanes whose row is at or past L, or whose 8 k start at or past L,
// load zeros (rows past L are never written; k past L is zero up to the 8-aligned edge).
// Same MFMAs in the same order as tmu_contract_kernel: the same bits. The output tile is
// staged per wave in LDS and leaves as whole 128-byte row segments.
namespace {
constexpr int NSF = 3;             // k-steps in flight per wave
constexpr int FSR = 64 + 8;        // per-wave staging row stride (halfs)
}  // namespace

__global__ __launch_bounds__(256, 2) void tmu_contract_frag_kernel(ContractArgs p) {
  __shared__ __align__(16) half_t stg[4][64 * FSR];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wr = wave >> 1, wc = wave & 1;
  const int L = p.L;
  const int rbn = (L + 31) / 32, kbn = (L + 15) / 16;
  const int nb = (rbn + 3) / 4;                    // 128-row blocks per dimension
  const int t = xcd_remap(blockIdx.x, gridDim.x);  // a channel's nb^2 blocks share an L2
  const int ch = t / (nb * nb), rem = t - ch * nb * nb;
  const int bi = rem / nb, bj = rem - bi * nb;
  const int rb0 = (bi * 2 + wr) * 2, cb0 = (bj * 2 + wc) * 2;  // first 32-row block of A and of B
  const size_t plane = (size_t)rbn * kbn * FragLayout::kTileHalfs;
  const rsrc_t rA = make_rsrc(p.a + (size_t)ch * plane), rB = make_rsrc(p.b + (size_t)ch * plane);
  const int lr = lane & 31, lk = 8 * (lane >> 5);
  auto toff = [&](int rb, int kb) -> uint32_t {
    const bool ok = rb < rbn && 32 * rb + lr < L && kb < kbn && 16 * kb + lk < L;
    return ok ? (uint32_t)((((size_t)rb * kbn + kb) * 64 + lane) * 16) : kOOB;
  };
  f32x16 acc[2][2];
#pragma unroll
  for (int u = 0; u < 2; u++)
#pragma unroll
    for (int v = 0; v < 2; v++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[u][v][e] = 0.f;
  half8 fa[NSF][2], fb[NSF][2];
#pragma unroll
  for (int st = 0; st < NSF; st++)
#pragma unroll
    for (int u = 0; u < 2; u++) {
      fa[st][u] = bload16(rA, toff(rb0 + u, st));
      fb[st][u] = bload16(rB, toff(cb0 + u, st));
    }
  // k-steps past kbn load zeros and add nothing; the loop runs a whole number of rounds
  const int nk = (kbn + NSF - 1) / NSF * NSF;
  for (int k0 = 0; k0 < nk; k0 += NSF) {
#pragma unroll
    for (int st = 0; st < NSF; st++) {
#pragma unroll
      for (int u = 0; u < 2; u++)
#pragma unroll
        for (int v = 0; v < 2; v++) acc[u][v] = mfma32(fb[st][v], fa[st][u], acc[u][v]);  // D[j][i]
#pragma unroll
      for (int u = 0; u < 2; u++) {
        fa[st][u] = bload16(rA, toff(rb0 + u, k0 + NSF + st));
        fb[st][u] = bload16(rB, toff(cb0 + u, k0 + NSF + st));
      }
    }
  }
  // lane: i = 32u + lane % 32, j = 32v + 8g + 4 (lane / 32) .. +3
  half_t* sw = stg[wave];
#pragma unroll
  for (int u = 0; u < 2; u++)
#pragma unroll
    for (int v = 0; v < 2; v++)
#pragma unroll
      for (int g = 0; g < 4; g++) {
        half4 h;
#pragma unroll
        for (int e = 0; e < 4; e++) h[e] = (half_t)(acc[u][v][4 * g + e] * p.scale);
        *reinterpret_cast<half4*>(sw + (32 * u + lr) * FSR + acc_row32(4 * g, lane) + 32 * v) = h;
      }
  // the staging rows are private to the wave; this keeps the reads below the writes
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const int i0 = 32 * rb0, j0 = 32 * cb0;
  const rsrc_t rX = make_rsrc(p.x + ((size_t)ch * L) * p.ldx);
#pragma unroll
  for (int q = 0; q < 8; q++) {
    const int row = 8 * q + (lane >> 3), chunk = lane & 7;
    const int i = i0 + row, j = j0 + 8 * chunk;
    const bool ok = i < L && j < p.ldx;
    bstore16(rX, ok ? (uint32_t)((size_t)i * p.ldx + j) * 2u : kOOB, ld16(sw + row * FSR + 8 * chunk));
  }
}

hipError_t launch_contract(const ContractArgs& a, hipStream_t s) {
  if (a.frag) {
    const int nb = ((a.L + 31) / 32 + 3) / 4;
    ESM_LAUNCH(tmu_contract_frag_kernel, dim3((unsigned)((long long)a.batch * nb * nb)), dim3(256), 0, s, a);
    return hipGetLastError();
  }
  const long long blocks = (long long)a.batch * ((a.L + BM - 1) / BM) * ((a.L + BN - 1) / BN);
  ESM_LAUNCH(tmu_contract_kernel, dim3((unsigned)blocks), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace esm
