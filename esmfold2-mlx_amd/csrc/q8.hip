// Kernel (d): MLX-affine 8-bit weight-only linear, y = x . W^T, with
// W[n, k] = RN_fp16(s[n, k/64] * q[n, k] + b[n, k/64]), fp32 accumulation on
// MFMA, one rounding of y to fp16.
//
// Dequantisation, 3 packed instructions per 2 codes: v_perm_b32 puts a code byte
// under the fp16 exponent of 1024 (bits 0x64qq = 1024 + q, exact), v_pk_add_f16
// subtracts 1024 (exact: q), v_pk_fma_f16 gives RN(s*q + b) with one rounding. The
// same bits as the dequantise entry point.
//
// Tiling: a workgroup owns a 64 (m) x 32 NB (n) tile of y = 2 x NB blocks of the
// 32x32x16 MFMA (NB = 5, 160 rows, or 4, 128 rows: the launch plan picks the width that
// fills the GPU in the fewest rounds), and a range of K, walked in steps of two 64-wide
// groups (128 k). Each step's codes (32 NB rows x 128 B), x (64 rows x 256 B) and packed
// scales are loaded with row-contiguous 16-byte loads (8 or 16 lanes per row, one step
// ahead in registers) and stored to one of two LDS stages; one barrier per step. Wave w
// then takes MFMA step kk = w of both groups: every wave accumulates the whole tile (2 NB
// independent chains) over its quarter of each step's k, so every dequantised weight
// feeds 64 rows of x and no two waves dequantise the same weight. Each output's sum runs
// over the same k in the same order at either width: the same bits. (Loading the MFMA
// fragments straight from global memory instead puts 32 rows in every load
// instruction, i.e. 32 to 64 cache lines for 1 KB, and measured 1.8x slower.)
// Weight codes dominate the traffic (1 byte per MAC row); M-tiles of the same n-tile
// are neighbours in the XCD-aware order and read the codes from one L2.
//
// The tile's 4 partial sums meet in LDS. When K is split over several workgroups
// (small grids: M x N too small to fill the GPU), each writes an fp32 partial to the
// caller's workspace and a second kernel sums the partials in split order (the kernel
// boundary orders the writes before the reads; no fences or counters): the result does
// not depend on the order the workgroups ran in. That second kernel is either the
// reduction here or, for a linear whose output feeds a residual + LayerNorm, the
// LayerNorm itself (esmc_ln_kernel sums the same partials in the same order).
#include <mutex>

#include "common.h"
#include "kernels.h"

namespace esm {

namespace {
constexpr int QG = 64;           // quantisation group: k per step
constexpr int MBQ = 2;           // 32-row m blocks per tile
constexpr int NWQ = 4;           // waves per workgroup
static_assert(kQ8TileM == 32 * MBQ && kQ8Waves == NWQ, "tile geometry");
}  // namespace

DEV uint32_t perm_b32(uint32_t hi, uint32_t lo, uint32_t sel) { return __builtin_amdgcn_perm(hi, lo, sel); }

// 8 codes (little-endian bytes of lo, hi) -> 8 fp16 weights RN(s*q + b).
DEV half8 dequant8(uint32_t lo, uint32_t hi, half2v s2, half2v b2) {
  // v_perm_b32 selector bytes 0-3 pick from the second operand (the codes), 4 picks
  // 0x64 from the first: [q0, 0x64, q1, 0x64] is the fp16 pair (1024 + q0, 1024 + q1).
  constexpr uint32_t kExp = 0x64646464u, kSel01 = 0x04010400u, kSel23 = 0x04030402u;
  const uint32_t h[4] = {perm_b32(kExp, lo, kSel01), perm_b32(kExp, lo, kSel23), perm_b32(kExp, hi, kSel01),
                         perm_b32(kExp, hi, kSel23)};
  const half2v k1024 = {(half_t)1024.0f, (half_t)1024.0f};
  half8 out;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const half2v qv = __builtin_bit_cast(half2v, h[i]) - k1024;  // exact
    const half2v w = __builtin_elementwise_fma(qv, s2, b2);      // one rounding of s*q + b
    out[2 * i] = w[0];
    out[2 * i + 1] = w[1];
  }
  return out;
}

DEV half2v splat2(uint32_t bits) {
  const half_t v = __builtin_bit_cast(half_t, (uint16_t)bits);
  return half2v{v, v};
}

// LDS stage of one step (two groups, 128 k) of a tile. Codes: TN rows of 128 B at a
// 136-byte stride (rows start on 32 distinct even banks: the 8-byte fragment reads of
// 32 rows are conflict-free); x: 64 rows of 256 B at a 272-byte stride (16 rows per
// 16-byte read pass on distinct banks); scale/bias pairs packed (b << 16 | s) per group.
constexpr int QSTR = 136, XSTR = 272;
constexpr int NT = NWQ * 64;
constexpr int XSTAGE = kQ8TileM * XSTR;
constexpr int XCH = kQ8TileM * 16 / NT;  // 16-byte x chunks per thread per step (4)
template <int NB>
struct Q8Geo {
  static constexpr int TN = 32 * NB;                       // weight rows per tile
  static constexpr int NBLK = MBQ * NB;                    // accumulator blocks per tile
  static constexpr int QSTAGE = TN * QSTR, SBSTAGE = 2 * TN * 4;
  static constexpr int STAGE = QSTAGE + XSTAGE + SBSTAGE;
  static constexpr int QCH = TN * 8 / NT;                  // 16-byte code chunks per thread per step
  static constexpr int RED_BYTES = NWQ * NBLK * 4 * 64 * 16;
  static constexpr int SBT = 16 * NB;                      // threads that load a step's packed scale words
  static_assert(TN * 8 % NT == 0 && kQ8TileM * 16 % NT == 0 && TN <= NT && SBT <= NT, "loader split");
  static_assert(2 * STAGE <= RED_BYTES, "stages fit in the reduction area");
};

// One step's global loads of one thread (registers, issued a step ahead of their LDS store).
template <int NB>
struct Q8Load {
  u32x4 q[Q8Geo<NB>::QCH];
  u32x4 x[XCH];
  u32x4 sbv;                  // packed scales: 4 (b << 16 | s) words of the step's 64 NB
  uint32_t s0, s1, b0, b1;    // unpacked: one row's two groups
};

// Packed scales [N/32][K/64][32] words: a step's two groups of one 32-row block are 64
// consecutive words. Thread i < 16 NB loads 4 of them: block i / 16, group i % 16 / 8,
// rows 4 (i % 8) .. + 3. Its byte offset from the tile's first block (kOOB for the second
// group of a step that has one), and where the words go in the [2][TN] LDS stage.
DEV uint32_t sb_offset(int i, int g, int ngroups, bool two) {
  const int nb = i >> 4, pc = i & 15;
  return (pc < 8 || two) ? (((uint32_t)nb * ngroups + g) * 32u + 4u * pc) * 4u : kOOB;
}
template <int NB>
DEV int sb_slot(int i) {
  return ((i & 15) >> 3) * Q8Geo<NB>::TN + 32 * (i >> 4) + 4 * (i & 7);
}

// PACKED: scales and biases come pre-packed per 32-row block ([N/32][group][32] words of
// b << 16 | s, from q8_pack_scales): a step's words of one block are 256 contiguous bytes,
// one 16-byte load for 16 threads. Unpacked, every thread of the first TN reads its row's
// fp16 pairs from the [N, K/64] arrays: TN scattered rows per step, several times the
// L1 requests of the codes and x together.
//
// PCODES: the codes come packed by q8_pack_codes, each MFMA A-fragment's 8 codes of both groups
// of a step next to each other for its lane: a wave loads its NB fragments of a step as NB fully
// coalesced 1 KB loads straight into registers (two steps ahead), and only x and the scales
// pass through LDS (43 instead of 73 KB of LDS traffic per step at NB = 5). Same MFMAs in the
// same order: the same bits as the [N, K] codes.
template <bool PACKED, bool PCODES, int NB>
__global__ __launch_bounds__(NWQ * 64, 1) void q8_linear_kernel(Q8Args p) {
  static_assert(PACKED || !PCODES, "packed codes are read with packed scales");
  using G = Q8Geo<NB>;
  constexpr int TN = G::TN, NBLK = G::NBLK, QSTAGE = G::QSTAGE, STAGE = G::STAGE, QCH = G::QCH, SBT = G::SBT;
  __shared__ __align__(16) char smem[G::RED_BYTES];  // two step stages, then every wave's partial tile

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 31, kg = lane >> 5;

  // Logical order: split slowest, then n-tile, then m-tile fastest. XCD neighbours share
  // codes (the m-tiles of one n-tile), and each K-split's workgroups fill whole XCDs, so
  // a K-slice of x is fetched by the L2s of those XCDs only.
  int t = xcd_remap(blockIdx.x, gridDim.x);
  const int mt = t % p.mtiles;
  t /= p.mtiles;
  const int nt = t % p.ntiles;
  const int sp = t / p.ntiles;
  const int m0 = mt * kQ8TileM, n0 = nt * TN;
  const int K = p.K, M = p.M, N = p.N, ngroups = K / QG;
  // This split's steps [st0, st1) of two groups each (whole steps, so a split starts where a
  // packed step does), i.e. groups [sg0, sg1).
  const int S = (ngroups + 1) / 2;
  const int st0 = (int)((long long)S * sp / p.splits), st1 = (int)((long long)S * (sp + 1) / p.splits);
  const int sg0 = 2 * st0, sg1 = 2 * st1 < ngroups ? 2 * st1 : ngroups;
  const int nsteps = st1 - st0;

  // Buffer ranges end exactly at the arrays' ends: rows past M or N load zeros. The
  // second group of a step past sg1 (odd group count) loads zeros for x, so it adds 0.
  // (Arrays a mode does not read get a descriptor of range 0 on x: the caller may pass NULL.)
  const rsrc_t rq = PCODES ? make_rsrc_n(p.x, 0u) : make_rsrc_n(p.q + (size_t)n0 * K, (uint32_t)(N - n0) * (uint32_t)K);
  const rsrc_t rs = PACKED ? make_rsrc_n(p.x, 0u)
                           : make_rsrc_n(p.s + (size_t)n0 * ngroups, (uint32_t)(N - n0) * (uint32_t)ngroups * 2u);
  const rsrc_t rb = PACKED ? make_rsrc_n(p.x, 0u)
                           : make_rsrc_n(p.b + (size_t)n0 * ngroups, (uint32_t)(N - n0) * (uint32_t)ngroups * 2u);
  const rsrc_t rx = make_rsrc_n(p.x + (size_t)m0 * K, (uint32_t)(M - m0) * (uint32_t)K * 2u);
  // the tile's blocks of the packed layouts (blocks past N are out of range: zeros)
  const int blk0 = n0 / 32, nblk = (N + 31) / 32 - blk0 < NB ? (N + 31) / 32 - blk0 : NB;
  const rsrc_t rsb = make_rsrc_n(PACKED ? (const void*)(p.sb + (size_t)blk0 * ngroups * 32) : (const void*)p.x,
                                 PACKED ? (uint32_t)nblk * (uint32_t)ngroups * 128u : 0u);

  // Coalesced loads: 8 lanes per 128-byte code row piece, 16 lanes per 256-byte x row piece.
  auto gload = [&](Q8Load<NB>& ld, int step) {
    const int g = sg0 + 2 * step;
    const bool two = g + 1 < sg1;
#pragma unroll
    for (int i = 0; i < QCH; i++) {
      const int c = tid + NT * i, row = c >> 3, j = c & 7;
      ld.q[i] = __builtin_amdgcn_raw_buffer_load_b128(rq, (int)((uint32_t)row * K + g * QG + 16 * j), 0, 0);
    }
#pragma unroll
    for (int i = 0; i < XCH; i++) {
      const int c = tid + NT * i, row = c >> 4, j = c & 15;
      const uint32_t off = (j < 8 || two) ? ((uint32_t)row * K + g * QG) * 2u + 16u * j : kOOB;
      ld.x[i] = __builtin_amdgcn_raw_buffer_load_b128(rx, (int)off, 0, 0);
    }
    if (PACKED) {
      ld.sbv = __builtin_amdgcn_raw_buffer_load_b128(rsb, (int)(tid < SBT ? sb_offset(tid, g, ngroups, two) : kOOB), 0, 0);
    } else {
      const uint32_t so = tid < TN ? ((uint32_t)tid * ngroups + g) * 2u : kOOB;
      ld.s0 = bload2(rs, so);
      ld.s1 = bload2(rs, so + 2u);
      ld.b0 = bload2(rb, so);
      ld.b1 = bload2(rb, so + 2u);
    }
  };
  auto sstore = [&](const Q8Load<NB>& ld, int buf) {
    char* st = smem + buf * STAGE;
#pragma unroll
    for (int i = 0; i < QCH; i++) {
      const int c = tid + NT * i, row = c >> 3, j = c & 7;
      u32x2* d = reinterpret_cast<u32x2*>(st + row * QSTR + 16 * j);  // 8-byte aligned rows
      d[0] = u32x2{ld.q[i][0], ld.q[i][1]};
      d[1] = u32x2{ld.q[i][2], ld.q[i][3]};
    }
#pragma unroll
    for (int i = 0; i < XCH; i++) {
      const int c = tid + NT * i, row = c >> 4, j = c & 15;
      *reinterpret_cast<u32x4*>(st + QSTAGE + row * XSTR + 16 * j) = ld.x[i];
    }
    uint32_t* sb = reinterpret_cast<uint32_t*>(st + QSTAGE + XSTAGE);
    if (PACKED) {
      if (tid < SBT) *reinterpret_cast<u32x4*>(sb + sb_slot<NB>(tid)) = ld.sbv;
    } else if (tid < TN) {
      sb[tid] = (ld.b0 << 16) | (ld.s0 & 0xffffu);
      sb[TN + tid] = (ld.b1 << 16) | (ld.s1 & 0xffffu);
    }
  };

  f32x16 acc[MBQ][NB];
#pragma unroll
  for (int mb = 0; mb < MBQ; mb++)
#pragma unroll
    for (int nb = 0; nb < NB; nb++)
#pragma unroll
      for (int i = 0; i < 16; i++) acc[mb][nb][i] = 0.f;

  // Wave w takes MFMA step kk = w (k = 16 w .. 16 w + 15) of both groups of a step:
  // D[n][m] += W[n][k] x[m][k], A = dequantised codes (row n = lane%32), B = x.
  auto compute = [&](int buf) {
    const char* st = smem + buf * STAGE;
    const uint32_t* sb = reinterpret_cast<const uint32_t*>(st + QSTAGE + XSTAGE);
#pragma unroll
    for (int g = 0; g < 2; g++) {
      half8 a[NB];
#pragma unroll
      for (int nb = 0; nb < NB; nb++) {
        const int row = 32 * nb + r;
        const uint32_t w = sb[g * TN + row];
        const u32x2 c = *reinterpret_cast<const u32x2*>(st + row * QSTR + 64 * g + 16 * wave + 8 * kg);
        a[nb] = dequant8(c[0], c[1], splat2(w & 0xffffu), splat2(w >> 16));
      }
      half8 xf[MBQ];
#pragma unroll
      for (int mb = 0; mb < MBQ; mb++)
        xf[mb] = *reinterpret_cast<const half8*>(st + QSTAGE + (32 * mb + r) * XSTR + 128 * g + 32 * wave + 16 * kg);
#pragma unroll
      for (int nb = 0; nb < NB; nb++)
#pragma unroll
        for (int mb = 0; mb < MBQ; mb++) acc[mb][nb] = mfma32(a[nb], xf[mb], acc[mb][nb]);
    }
  };

  if constexpr (!PCODES) {
    // Pipeline: step s+2's loads in flight while step s computes from LDS and step s+1's
    // registers wait to be stored; one barrier per step. Unrolled by two (register sets
    // A and B), a single loop exit, the leftover step after it.
    Q8Load<NB> la, lb;
    if (nsteps > 0) {
      gload(la, 0);
      gload(lb, 1);
      sstore(la, 0);
      __syncthreads();
    }
    int st = 0;
    for (; st + 2 <= nsteps; st += 2) {
      gload(la, st + 2);
      compute(0);
      sstore(lb, 1);
      __syncthreads();
      gload(lb, st + 3);
      compute(1);
      sstore(la, 0);
      __syncthreads();
    }
    if (st < nsteps) compute(0);
  } else {
    // Codes of step s (this wave's NB fragments) in register set A or B from two steps before;
    // x and the scales staged as above, in a stage without the codes area. Packed codes
    // [N/32][S][4 waves][64 lanes][16 B]: fragment nb of a step is 1 KB at block blk0 + nb.
    constexpr int XS = XSTAGE + G::SBSTAGE;
    constexpr uint32_t kWaveStep = NWQ * 1024;  // one step of one 32-row block
    const rsrc_t rqp = make_rsrc_n(p.qp + (size_t)blk0 * S * kWaveStep, (uint32_t)nblk * (uint32_t)S * kWaveStep);
    auto gcodes = [&](u32x4 (&cq)[NB], int step) {
#pragma unroll
      for (int nb = 0; nb < NB; nb++)
        cq[nb] = __builtin_amdgcn_raw_buffer_load_b128(
            rqp,
            (int)(step < nsteps ? ((uint32_t)nb * S + st0 + step) * kWaveStep + (uint32_t)(wave * 1024 + lane * 16) : kOOB),
            0, 0);
    };
    auto xload = [&](u32x4 (&xv)[XCH], u32x4& sbv, int step) {
      const int g = sg0 + 2 * step;
      const bool two = g + 1 < sg1;
#pragma unroll
      for (int i = 0; i < XCH; i++) {
        const int c = tid + NT * i, row = c >> 4, j = c & 15;
        const uint32_t off = (j < 8 || two) ? ((uint32_t)row * K + g * QG) * 2u + 16u * j : kOOB;
        xv[i] = __builtin_amdgcn_raw_buffer_load_b128(rx, (int)off, 0, 0);
      }
      sbv = __builtin_amdgcn_raw_buffer_load_b128(rsb, (int)(tid < SBT ? sb_offset(tid, g, ngroups, two) : kOOB), 0, 0);
    };
    auto xstore = [&](const u32x4 (&xv)[XCH], const u32x4& sbv, int buf) {
      char* st = smem + buf * XS;
#pragma unroll
      for (int i = 0; i < XCH; i++) {
        const int c = tid + NT * i, row = c >> 4, j = c & 15;
        *reinterpret_cast<u32x4*>(st + row * XSTR + 16 * j) = xv[i];
      }
      if (tid < SBT) *reinterpret_cast<u32x4*>(reinterpret_cast<uint32_t*>(st + XSTAGE) + sb_slot<NB>(tid)) = sbv;
    };
    auto compute_pc = [&](int buf, const u32x4 (&cq)[NB]) {
      const char* st = smem + buf * XS;
      const uint32_t* sb = reinterpret_cast<const uint32_t*>(st + XSTAGE);
#pragma unroll
      for (int g = 0; g < 2; g++) {
        half8 a[NB];
#pragma unroll
        for (int nb = 0; nb < NB; nb++) {
          const uint32_t w = sb[g * TN + 32 * nb + r];
          a[nb] = dequant8(cq[nb][2 * g], cq[nb][2 * g + 1], splat2(w & 0xffffu), splat2(w >> 16));
        }
        half8 xf[MBQ];
#pragma unroll
        for (int mb = 0; mb < MBQ; mb++)
          xf[mb] = *reinterpret_cast<const half8*>(st + (32 * mb + r) * XSTR + 128 * g + 32 * wave + 16 * kg);
#pragma unroll
        for (int nb = 0; nb < NB; nb++)
#pragma unroll
          for (int mb = 0; mb < MBQ; mb++) acc[mb][nb] = mfma32(a[nb], xf[mb], acc[mb][nb]);
      }
    };
    u32x4 xa[XCH], xb[XCH], sa, sbb, ca[NB], cb[NB];
    if (nsteps > 0) {
      xload(xa, sa, 0);
      gcodes(ca, 0);
      xload(xb, sbb, 1);
      gcodes(cb, 1);
      xstore(xa, sa, 0);
      __syncthreads();
    }
    int st = 0;
    for (; st + 2 <= nsteps; st += 2) {
      xload(xa, sa, st + 2);
      compute_pc(0, ca);
      gcodes(ca, st + 2);
      xstore(xb, sbb, 1);
      __syncthreads();
      xload(xb, sbb, st + 3);
      compute_pc(1, cb);
      gcodes(cb, st + 3);
      xstore(xa, sa, 0);
      __syncthreads();
    }
    if (st < nsteps) compute_pc(0, ca);
  }
  __syncthreads();  // the stages are reused as the reduction area

  // The 4 partial tiles -> LDS; wave w then finishes blocks w, w+4, w+8.
  f32x4 (*red)[NBLK][4][64] = reinterpret_cast<f32x4 (*)[NBLK][4][64]>(smem);
#pragma unroll
  for (int mb = 0; mb < MBQ; mb++)
#pragma unroll
    for (int nb = 0; nb < NB; nb++)
#pragma unroll
      for (int r4 = 0; r4 < 4; r4++)
        red[wave][mb * NB + nb][r4][lane] =
            f32x4{acc[mb][nb][4 * r4], acc[mb][nb][4 * r4 + 1], acc[mb][nb][4 * r4 + 2], acc[mb][nb][4 * r4 + 3]};
  __syncthreads();

  // Lane's output coordinates in block blk: column m = lane%32, rows n = 4 consecutive per r4.
  auto tile_sum = [&](int blk, int r4) {
    f32x4 v = red[0][blk][r4][lane];
#pragma unroll
    for (int w = 1; w < NWQ; w++) v += red[w][blk][r4][lane];
    return v;
  };
  if constexpr (NB == kQ8TileNbWide) if (p.part == nullptr && p.swiglu) {
    // SwiGLU pairs (160-row tiles only): a lane's 4 gate rows n .. n+3 (n = 32 nb + 8 r4 + 4 h
    // < 80) have their up rows at n + 80 = 32 (nb + 2) + 8 (r4 + 2) + 4 h: the same lane's sums
    // in block nb + 2 or nb + 3. Both round to fp16 as y would, then silu(gate) * up in fp32 as esmc_swiglu does.
    constexpr int HALF = kQ8SwigluHalf, NG = MBQ * HALF / 8;  // gate groups of 8 rows per tile
    const int F = N / 2;
    for (int gi = wave; gi < NG; gi += NWQ) {
      const int mb = gi / (HALF / 8), g8 = gi - mb * (HALF / 8);  // gate rows 8 g8 .. 8 g8 + 7
      const int nb = g8 >> 2, r4 = g8 & 3;
      const int ru = r4 + 2, nbu = nb + 2 + (ru >> 2);
      const f32x4 g = tile_sum(mb * NB + nb, r4), u = tile_sum(mb * NB + nbu, ru & 3);
      const int m = m0 + 32 * mb + r, f = nt * HALF + 8 * g8 + 4 * kg;
      half4 o;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const float a = (float)(half_t)g[e];
        o[e] = (half_t)(a * sigmoidf_fast(a) * (float)(half_t)u[e]);
      }
      if (m < M && f < F) *reinterpret_cast<half4*>(p.y + (size_t)m * F + f) = o;
    }
    return;
  }
  if (p.part == nullptr) {  // one K range per tile: fp16 y directly
    for (int blk = wave; blk < NBLK; blk += NWQ) {
      const int mb = blk / NB, nb = blk - mb * NB;
      const int m = m0 + 32 * mb + r;
#pragma unroll
      for (int r4 = 0; r4 < 4; r4++) {
        const int n = n0 + 32 * nb + acc_row32(4 * r4, lane);
        const f32x4 v = tile_sum(blk, r4);
        if (m < M && n < N)
          *reinterpret_cast<half4*>(p.y + (size_t)m * N + n) = half4{(half_t)v[0], (half_t)v[1], (half_t)v[2], (half_t)v[3]};
      }
    }
    return;
  }

  // This workgroup's fp32 partial (split sp of p.splits, possibly the only one); q8_reduce_kernel
  // or the consumer (esmc_ln_kernel) sums the splits.
  float* part = p.part + (size_t)sp * M * N;
  for (int blk = wave; blk < NBLK; blk += NWQ) {
    const int mb = blk / NB, nb = blk - mb * NB;
    const int m = m0 + 32 * mb + r;
#pragma unroll
    for (int r4 = 0; r4 < 4; r4++) {
      const int n = n0 + 32 * nb + acc_row32(4 * r4, lane);
      const f32x4 v = tile_sum(blk, r4);
      if (m < M && n < N) *reinterpret_cast<f32x4*>(part + (size_t)m * N + n) = v;
    }
  }
}

// y = sum of the split partials in split order (deterministic), one rounding to fp16.
// Four outputs per thread; M * N is a multiple of 64.
__global__ __launch_bounds__(256) void q8_reduce_kernel(const float* __restrict__ part, half_t* __restrict__ y,
                                                        size_t n4, size_t plane, int splits) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (size_t)gridDim.x * blockDim.x) {
    f32x4 v = reinterpret_cast<const f32x4*>(part)[i];
    for (int s = 1; s < splits; s++) v += reinterpret_cast<const f32x4*>(part + (size_t)s * plane)[i];
    reinterpret_cast<half4*>(y)[i] = half4{(half_t)v[0], (half_t)v[1], (half_t)v[2], (half_t)v[3]};
  }
}

// The same for SwiGLU pair rows: out [M, F] = silu(gate) * up, each of gate and up summed over
// the splits in order and rounded to fp16 first (the bits of the fused epilogue). Four outputs
// per thread; F is a multiple of 80.
__global__ __launch_bounds__(256) void q8_reduce_swiglu_kernel(const float* __restrict__ part,
                                                               half_t* __restrict__ y, int M, int F, int splits) {
  const size_t plane = (size_t)M * 2 * F, n4 = (size_t)M * F / 4;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (size_t)gridDim.x * blockDim.x) {
    const size_t m = 4 * i / F;
    const int f = (int)(4 * i - m * F);
    const int cg = 2 * kQ8SwigluHalf * (f / kQ8SwigluHalf) + f % kQ8SwigluHalf;  // gate column
    const float* pg = part + m * 2 * F + cg;
    f32x4 g = *reinterpret_cast<const f32x4*>(pg), u = *reinterpret_cast<const f32x4*>(pg + kQ8SwigluHalf);
    for (int s = 1; s < splits; s++) {
      g += *reinterpret_cast<const f32x4*>(pg + s * plane);
      u += *reinterpret_cast<const f32x4*>(pg + s * plane + kQ8SwigluHalf);
    }
    half4 o;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const float a = (float)(half_t)g[e];
      o[e] = (half_t)(a * sigmoidf_fast(a) * (float)(half_t)u[e]);
    }
    *reinterpret_cast<half4*>(y + 4 * i) = o;
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
    const size_t gi = n * (K / QG) + k / QG;
    const u32x4 v = *reinterpret_cast<const u32x4*>(q + e0);
    const half2v s2 = splat2(__builtin_bit_cast(uint16_t, s[gi])), b2 = splat2(__builtin_bit_cast(uint16_t, b[gi]));
    st16(w + e0, dequant8(v[0], v[1], s2, b2));
    st16(w + e0 + 8, dequant8(v[2], v[3], s2, b2));
  }
}

// sb[(j * ngroups + g) * 32 + r] = b[n, g] << 16 | s[n, g] for n = 32 j + r (0 past N): per
// 32-row block, so a tile of any whole number of blocks reads its words at one base.
__global__ __launch_bounds__(256) void q8_pack_kernel(const uint16_t* __restrict__ s, const uint16_t* __restrict__ b,
                                                      uint32_t* __restrict__ sb, int N, int ngroups, size_t total) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const int r = (int)(i % 32);
    const size_t rest = i / 32;
    const int g = (int)(rest % ngroups);
    const int n = (int)(rest / ngroups) * 32 + r;
    sb[i] = n < N ? ((uint32_t)b[(size_t)n * ngroups + g] << 16) | s[(size_t)n * ngroups + g] : 0u;
  }
}

// Codes in the order q8_linear_kernel<true, true, NB> reads them: chunk ((j S + s) 4 + w),
// lane l, 16 bytes = the codes of row 32 j + l % 32 at k = 128 s + 16 w + 8 (l / 32) + 0..7
// (group 2s), then the same k + 64 (group 2s+1); zeros past N and past K. A 32-row block's
// steps are consecutive, so a tile of any whole number of blocks reads its fragments at one
// base. One thread per 16-byte chunk.
__global__ __launch_bounds__(256) void q8_pack_codes_kernel(const uint8_t* __restrict__ q, uint8_t* __restrict__ qp,
                                                            int N, int K, size_t nchunks) {
  const int S = (K / QG + 1) / 2;
  for (size_t c = (size_t)blockIdx.x * blockDim.x + threadIdx.x; c < nchunks; c += (size_t)gridDim.x * blockDim.x) {
    const int lane = (int)(c % 64);
    size_t rest = c / 64;
    const int w = (int)(rest % NWQ);
    rest /= NWQ;
    const int s = (int)(rest % S);
    const int j = (int)(rest / S);
    const int n = 32 * j + (lane & 31);
    const int k0 = 128 * s + 16 * w + 8 * (lane >> 5);
    u32x2 lo = {0u, 0u}, hi = {0u, 0u};
    if (n < N) {
      lo = *reinterpret_cast<const u32x2*>(q + (size_t)n * K + k0);
      if (k0 + 64 < K) hi = *reinterpret_cast<const u32x2*>(q + (size_t)n * K + k0 + 64);
    }
    *reinterpret_cast<u32x4*>(qp + c * 16) = u32x4{lo[0], lo[1], hi[0], hi[1]};
  }
}

hipError_t launch_q8_pack_codes(const uint8_t* q, uint8_t* qp, int N, int K, hipStream_t st) {
  const size_t nchunks = q8_packed_codes_size(N, K) / 16;
  const size_t blocks = (nchunks + 255) / 256;
  ESM_LAUNCH(q8_pack_codes_kernel, dim3((unsigned)(blocks < 4096 ? blocks : 4096)), dim3(256), 0, st, q, qp, N, K,
             nchunks);
  return hipGetLastError();
}

hipError_t launch_q8_pack(const half_t* s, const half_t* b, uint32_t* sb, int N, int K, hipStream_t st) {
  const int ngroups = K / QG;
  const size_t total = q8_packed_scales_words(N, K);
  const size_t blocks = (total + 255) / 256;
  ESM_LAUNCH(q8_pack_kernel, dim3((unsigned)(blocks < 4096 ? blocks : 4096)), dim3(256), 0, st,
                     reinterpret_cast<const uint16_t*>(s), reinterpret_cast<const uint16_t*>(b), sb, N, ngroups, total);
  return hipGetLastError();
}

// ---- device scratch of the allocation-free entry point -----------------------------------
// q8_linear_noalloc runs the same plan as q8_linear_ws with its split-K partials in this
// file-scope array instead of a caller workspace: kQ8ScratchBytes per device, held for the
// life of the process. On the host, `scratch` names a host-side stand-in, never the device
// memory: its device address is taken once per device with hipGetSymbolAddress (with that
// device current) and only that address reaches a kernel. Every split writes all of its
// partial outputs before the reduction reads them, so nothing needs clearing between calls;
// calls that overlap in time on one device share the array and race.
static __device__ __align__(256) float scratch[kQ8ScratchBytes / sizeof(float)];

hipError_t q8_scratch_address(float** ptr) {
  constexpr int kMaxDev = 64;
  static std::mutex mu;
  static float* addr[kMaxDev] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDev) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(mu);
  if (addr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    addr[dev] = static_cast<float*>(p);
  }
  *ptr = addr[dev];
  return hipSuccess;
}

hipError_t launch_q8_linear(const Q8Args& a, hipStream_t s) {
  const int grid = a.mtiles * a.ntiles * a.splits;
  if (a.qp && !a.sb) return hipErrorInvalidValue;
  if (a.nb != kQ8TileNbWide && (a.nb != kQ8TileNbNarrow || a.swiglu)) return hipErrorInvalidValue;
#define Q8_LAUNCH(NB)                                                                  \
  if (a.qp)                                                                            \
    ESM_LAUNCH((q8_linear_kernel<true, true, NB>), dim3(grid), dim3(NWQ * 64), 0, s, a);  \
  else if (a.sb)                                                                       \
    ESM_LAUNCH((q8_linear_kernel<true, false, NB>), dim3(grid), dim3(NWQ * 64), 0, s, a); \
  else                                                                                 \
    ESM_LAUNCH((q8_linear_kernel<false, false, NB>), dim3(grid), dim3(NWQ * 64), 0, s, a);
  if (a.nb == kQ8TileNbWide) {
    Q8_LAUNCH(kQ8TileNbWide)
  } else {
    Q8_LAUNCH(kQ8TileNbNarrow)
  }
#undef Q8_LAUNCH
  if (a.part && a.y && a.swiglu) {  // partials of SwiGLU pair rows: summed and gated here
    const size_t n4 = (size_t)a.M * (a.N / 2) / 4, blocks = (n4 + 255) / 256;
    ESM_LAUNCH(q8_reduce_swiglu_kernel, dim3((unsigned)(blocks < 2048 ? blocks : 2048)), dim3(256), 0, s, a.part, a.y,
               a.M, a.N / 2, a.splits);
  } else if (a.part && a.y) {  // partials and an fp16 output: sum them here (no y: the caller's consumer does)
    const size_t plane = (size_t)a.M * a.N, n4 = plane / 4;
    const size_t blocks = (n4 + 255) / 256;
    ESM_LAUNCH(q8_reduce_kernel, dim3((unsigned)(blocks < 2048 ? blocks : 2048)), dim3(256), 0, s, a.part, a.y,
                       n4, plane, a.splits);
  }
  return hipGetLastError();
}

// MLX's affine 8-bit quantisation of fp32 weights W [N, K] along K, groups of 64 (the
// quantiser of layer_params, mlx_esmc.py:70-74): per group, scale = max((max - min) / 255,
// 1e-7) signed towards the larger-magnitude extreme (the edge), q0 = rint(edge / scale);
// unless q0 = 0 the scale becomes edge / q0 and the bias the edge (0 lands on the grid),
// else the bias is 0; codes clamp(rint((w - bias) / scale), 0, 255). fp32 arithmetic with
// IEEE division, rint = round half to even; scales and biases leave rounded to fp16.
// Sixteen lanes own one group (4 values each, one 16-byte load): min / max over the 16
// lanes, then 4 codes packed into one 4-byte store per lane.
__global__ __launch_bounds__(256) void q8_quantize_kernel(const float* __restrict__ w, uint8_t* __restrict__ q,
                                                          half_t* __restrict__ s, half_t* __restrict__ b,
                                                          size_t ngroups) {
  const int sub = threadIdx.x & 15;
  const size_t step = ((size_t)gridDim.x * blockDim.x) >> 4;
  for (size_t gi = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) >> 4; gi < ngroups; gi += step) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(w + gi * QG + 4 * sub);
    float lo = fminf(fminf(v[0], v[1]), fminf(v[2], v[3]));
    float hi = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
#pragma unroll
    for (int m = 8; m >= 1; m >>= 1) {  // the 16 lanes of this group only
      lo = fminf(lo, __shfl_xor(lo, m, 16));
      hi = fmaxf(hi, __shfl_xor(hi, m, 16));
    }
    const bool lo_edge = fabsf(lo) > fabsf(hi);
    float scale = fmaxf((hi - lo) / 255.0f, 1e-7f);
    scale = lo_edge ? scale : -scale;
    const float edge = lo_edge ? lo : hi;
    const float q0 = __builtin_rintf(edge / scale);
    const bool at_zero = q0 == 0.0f;
    scale = at_zero ? scale : edge / q0;
    const float bias = at_zero ? 0.0f : edge;
    uint32_t packed = 0;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const float c = fminf(fmaxf(__builtin_rintf((v[e] - bias) / scale), 0.0f), 255.0f);
      packed |= (uint32_t)c << (8 * e);
    }
    *reinterpret_cast<uint32_t*>(q + gi * QG + 4 * sub) = packed;
    if (sub == 0) {
      s[gi] = (half_t)scale;
      b[gi] = (half_t)bias;
    }
  }
}

hipError_t launch_q8_quantize(const float* w, uint8_t* q, half_t* s, half_t* b, int N, int K, hipStream_t st) {
  const size_t ngroups = (size_t)N * (K / QG);
  const size_t blocks = (ngroups * 16 + 255) / 256;
  const int grid = (int)(blocks < 8192 ? blocks : 8192);
  ESM_LAUNCH(q8_quantize_kernel, dim3(grid), dim3(256), 0, st, w, q, s, b, ngroups);
  return hipGetLastError();
}

hipError_t launch_q8_dequant(const uint8_t* q, const half_t* s, const half_t* b, half_t* w, int N, int K,
                             hipStream_t st) {
  const size_t nchunks = (size_t)N * K / 16;
  const size_t blocks = (nchunks + 255) / 256;
  const int grid = (int)(blocks < 4096 ? blocks : 4096);
  ESM_LAUNCH(q8_dequant_kernel, dim3(grid), dim3(256), 0, st, q, s, b, w, nchunks, K);
  return hipGetLastError();
}

}  // namespace esm
