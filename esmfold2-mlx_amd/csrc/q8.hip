// Kernel (d): MLX-affine 8-bit weight-only linear, y = x . W^T, with
// W[n, k] = RN_fp16(s[n, k/64] * q[n, k] + b[n, k/64]) computed by one packed
// fp16 FMA (v_pk_fma_f16: s*q is exact, so the result is the single rounding of
// the exact real value, the same bits as the dequantise entry point), fp32
// accumulation on MFMA, one rounding of y to fp16.
//
// Tiling: 64 (n) x 64 (m) outputs per workgroup, K in steps of one quantisation
// group (64). Per step the workgroup dequantises its 64x64 weight block into LDS
// once (each thread: 16 codes, one scale/bias pair) and stages the 64x64 x block;
// four waves (2x2) each run a 32x32 MFMA tile over the 4 k-substeps. Both LDS
// stages are double-buffered with register prefetch one step ahead.
// The MFMA computes y^T (rows n, columns m) so A = W and B = x are both
// k-contiguous rows; the 4 consecutive rows of an accumulator quad are 4
// consecutive n of one output row m: one 8-byte store.
#include "common.h"
#include "kernels.h"

namespace esm {

namespace {
constexpr int BN = 64;          // n per workgroup
constexpr int BM = 64;          // m per workgroup
constexpr int G = 64;           // quantisation group = k per step
constexpr int KS = G + 8;       // LDS row stride (halfs)
constexpr int WST = BN * KS;    // halfs per weight stage
constexpr int XST = BM * KS;    // halfs per x stage
}  // namespace

DEV half8 dequant8(uint32_t lo, uint32_t hi, half_t s, half_t b) {
  // 8 codes (little-endian bytes of lo, hi) -> 8 fp16 weights s*q + b, one rounding each.
  half8 q;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    q[e] = (half_t)(uint16_t)((lo >> (8 * e)) & 0xffu);
    q[e + 4] = (half_t)(uint16_t)((hi >> (8 * e)) & 0xffu);
  }
  half8 sv, bv;
#pragma unroll
  for (int e = 0; e < 8; e++) {
    sv[e] = s;
    bv[e] = b;
  }
  return __builtin_elementwise_fma(sv, q, bv);
}

__global__ __launch_bounds__(256, 2) void q8_linear_kernel(Q8Args p) {
  __shared__ __align__(16) half_t w_s[2 * WST];
  __shared__ __align__(16) half_t x_s[2 * XST];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int wn = wave >> 1, wm = wave & 1;
  const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
  const int K = p.K, M = p.M, ngroups = K / G;

  // Weight loader: thread -> (row n0 + tid/4, 16 codes at k = 16*(tid%4)).
  const int wrow = tid >> 2, wpart = tid & 3;
  const uint8_t* qrow = p.q + (size_t)(n0 + wrow) * K + wpart * 16;
  const half_t* srow = p.s + (size_t)(n0 + wrow) * ngroups;
  const half_t* brow = p.b + (size_t)(n0 + wrow) * ngroups;
  // x loader: 2 chunks of 8 halfs per thread.
  u32x4 qpre;
  half_t spre, bpre;
  half8 xpre[2];

  auto gload = [&](int kg) {
    qpre = *reinterpret_cast<const u32x4*>(qrow + (size_t)kg * G);
    spre = srow[kg];
    bpre = brow[kg];
#pragma unroll
    for (int u = 0; u < 2; u++) {
      const int id = tid + 256 * u;
      const int row = id >> 3, kc = id & 7;
      xpre[u] = (m0 + row < M) ? ld16(p.x + (size_t)(m0 + row) * K + (size_t)kg * G + kc * 8) : zero_half8();
    }
  };
  auto swrite = [&](int buf) {
    half_t* wd = w_s + buf * WST + wrow * KS + wpart * 16;
    st16(wd, dequant8(qpre[0], qpre[1], spre, bpre));
    st16(wd + 8, dequant8(qpre[2], qpre[3], spre, bpre));
#pragma unroll
    for (int u = 0; u < 2; u++) {
      const int id = tid + 256 * u;
      const int row = id >> 3, kc = id & 7;
      st16(x_s + buf * XST + row * KS + kc * 8, xpre[u]);
    }
  };

  f32x16 acc;
#pragma unroll
  for (int r = 0; r < 16; r++) acc[r] = 0.f;

  gload(0);
  swrite(0);
  __syncthreads();
  for (int kg = 0; kg < ngroups; kg++) {
    const int buf = kg & 1;
    if (kg + 1 < ngroups) gload(kg + 1);
    const half_t* ws = w_s + buf * WST + (wn * 32 + (lane & 31)) * KS + 8 * (lane >> 5);
    const half_t* xs = x_s + buf * XST + (wm * 32 + (lane & 31)) * KS + 8 * (lane >> 5);
#pragma unroll
    for (int kk = 0; kk < G / 16; kk++) acc = mfma32(ld16(ws + kk * 16), ld16(xs + kk * 16), acc);
    if (kg + 1 < ngroups) swrite(buf ^ 1);
    __syncthreads();
  }

  // acc rows are n, columns are m: 4 consecutive n per register quad.
  const int m = m0 + wm * 32 + (lane & 31);
  if (m < M) {
#pragma unroll
    for (int r4 = 0; r4 < 4; r4++) {
      const int n = n0 + wn * 32 + acc_row32(4 * r4, lane);
      half4 v;
#pragma unroll
      for (int e = 0; e < 4; e++) v[e] = (half_t)acc[4 * r4 + e];
      *reinterpret_cast<half4*>(p.y + (size_t)m * p.N + n) = v;
    }
  }
}

__global__ __launch_bounds__(256) void q8_dequant_kernel(const uint8_t* __restrict__ q, const half_t* __restrict__ s,
                                                         const half_t* __restrict__ b, half_t* __restrict__ w,
                                                         size_t nchunks, int K) {
  // One thread per 16 codes (16 | 64, so one scale/bias pair per chunk).
  for (size_t c = (size_t)blockIdx.x * blockDim.x + threadIdx.x; c < nchunks; c += (size_t)gridDim.x * blockDim.x) {
    const size_t e0 = c * 16;
    const size_t n = e0 / K;
    const size_t k = e0 - n * K;
    const size_t gi = n * (K / G) + k / G;
    const u32x4 v = *reinterpret_cast<const u32x4*>(q + e0);
    st16(w + e0, dequant8(v[0], v[1], s[gi], b[gi]));
    st16(w + e0 + 8, dequant8(v[2], v[3], s[gi], b[gi]));
  }
}

hipError_t launch_q8_linear(const Q8Args& a, hipStream_t s) {
  hipLaunchKernelGGL(q8_linear_kernel, dim3(a.N / BN, (a.M + BM - 1) / BM), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_q8_dequant(const uint8_t* q, const half_t* s, const half_t* b, half_t* w, int N, int K,
                             hipStream_t st) {
  const size_t nchunks = (size_t)N * K / 16;
  const size_t blocks = (nchunks + 255) / 256;
  const int grid = (int)(blocks < 4096 ? blocks : 4096);
  hipLaunchKernelGGL(q8_dequant_kernel, dim3(grid), dim3(256), 0, st, q, s, b, w, nchunks, K);
  return hipGetLastError();
}

}  // namespace esm
