// Kernels of the recycling step around the trunk (var_6b_mlx_loop.py:67-85,
// var_adaptive_loops.py:41-46, :109-118):
//   parcae_step          z <- a * z + LN(z_init + refined) @ B^T on every cell (fp32 state)
//   expected_distance    softmax((r + r^T) @ W^T + b) . centres per pair (distogram head)
//   abs_diff_quantile    the q-th quantile (linear interpolation) of |x - y| (exit signal)
// C = 128 pair channels.
#include "common.h"
#include "kernels.h"

namespace esm {

namespace {
constexpr int C = 128;
constexpr int NSTR = C + 8;  // LDS row stride (halfs) of a LayerNormed tile
}  // namespace

// ---- parcae step ----------------------------------------------------------------------------
// Persistent, 4 waves per workgroup; a tile is 32 consecutive cells. Wave w owns output
// channels [32w, 32w+32) and keeps those rows of B (fp16) as MFMA A fragments. Per tile:
// u = z_init + refined, LayerNorm (16 lanes per cell, fp32 statistics) into LDS as fp16,
// one barrier, D[co][cell] = B[co][:] . LN(u)[cell][:] (fp32 accumulation), then
// a[co] * z + D in fp32, 16-byte stores (4 consecutive channels per lane and quad).
__global__ __launch_bounds__(256, 1) void parcae_step_kernel(ParcaeArgs p) {
  __shared__ __align__(16) half_t n_s[32 * NSTR];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 31, h = lane >> 5;
  half8 bw[C / 16];
  {
    const half_t* row = p.b_mat + (size_t)(32 * wave + r) * C;
#pragma unroll
    for (int ks = 0; ks < C / 16; ks++) bw[ks] = ld16(row + 16 * ks + 8 * h);
  }
  const int ch0 = (lane & 15) * 8;
  float g[8], bb[8];
#pragma unroll
  for (int e = 0; e < 8; e++) {
    g[e] = p.ln_w[ch0 + e];
    bb[e] = p.ln_b[ch0 + e];
  }
  float av[16];  // a for this lane's 16 output channels
#pragma unroll
  for (int i = 0; i < 16; i++) av[i] = p.a[32 * wave + acc_row32(i, lane)];

  const rsrc_t rz = make_rsrc(p.z), ri = make_rsrc(p.z_init), rr = make_rsrc(p.refined), ro = make_rsrc(p.z_out);
  const size_t ncells = p.ncells;
  for (int tile = blockIdx.x; tile < p.ntiles; tile += gridDim.x) {
    const size_t cell0 = (size_t)tile * 32;
    // 1. u -> LayerNorm -> LDS
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int cl = (tid >> 4) + 16 * i;
      const uint32_t off = cell0 + cl < ncells ? (uint32_t)(((cell0 + cl) * C + ch0) * 4u) : kOOB;
      float v[8];
#pragma unroll
      for (int hh = 0; hh < 2; hh++) {
        const f32x4 a4 = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(ri, (int)(off + 16u * hh), 0, 0));
        const f32x4 b4 = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rr, (int)(off + 16u * hh), 0, 0));
#pragma unroll
        for (int e = 0; e < 4; e++) v[4 * hh + e] = a4[e] + b4[e];
      }
      ln_row128(v, g, bb, p.eps);
      half8 o;
#pragma unroll
      for (int e = 0; e < 8; e++) o[e] = (half_t)v[e];
      st16(&n_s[cl * NSTR + ch0], o);
    }
    __syncthreads();
    // 2. D[co][cell] over the wave's 32 output channels
    f32x16 d;
#pragma unroll
    for (int i = 0; i < 16; i++) d[i] = 0.f;
#pragma unroll
    for (int ks = 0; ks < C / 16; ks++) d = mfma32(bw[ks], ld16(&n_s[r * NSTR + 16 * ks + 8 * h]), d);
    // 3. a * z + D for the lane's cell and 4 quads of 4 consecutive channels
    const bool live = cell0 + r < ncells;
#pragma unroll
    for (int r4 = 0; r4 < 4; r4++) {
      const int co = 32 * wave + acc_row32(4 * r4, lane);
      const uint32_t off = live ? (uint32_t)(((cell0 + r) * C + co) * 4u) : kOOB;
      const f32x4 z4 = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rz, (int)off, 0, 0));
      f32x4 o;
#pragma unroll
      for (int e = 0; e < 4; e++) o[e] = av[4 * r4 + e] * z4[e] + d[4 * r4 + e];
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o), ro, (int)off, 0, 0);
    }
    __syncthreads();  // n_s is rewritten by the next tile
  }
}

// ---- expected distance ----------------------------------------------------------------------
// One wave per 32 pairs (b, i, j0 .. j0+31); 4 waves per workgroup. The B operand is
// s[cell][c] = r[b,i,j,c] + r[b,j,i,c] rounded to fp16, read straight into fragments
// (column = pair, k = channel); A = the head's weight rows (bins). A lane then holds its
// pair's logits for 16 bins per 32-bin block: the softmax over bins is a register
// reduction plus one exchange between the lane halves. Bias and centres come from LDS.
template <int NBB>  // 32-bin blocks
__global__ __launch_bounds__(256, 1) void expected_distance_kernel(DistoArgs p) {
  constexpr int NB = 32 * NBB;
  __shared__ float bias_s[NB], cent_s[NB];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 31, h = lane >> 5;
  for (int k = tid; k < NB; k += 256) {
    bias_s[k] = p.bias[k];
    cent_s[k] = p.centers[k];
  }
  half8 wa[NBB][C / 16];
#pragma unroll
  for (int bb = 0; bb < NBB; bb++)
#pragma unroll
    for (int ks = 0; ks < C / 16; ks++) wa[bb][ks] = ld16(p.w + (size_t)(32 * bb + r) * C + 16 * ks + 8 * h);
  __syncthreads();

  const int L = p.L;
  const int jt = (L + 127) / 128;  // 128-pair tiles per (b, i)
  for (int t = blockIdx.x; t < p.B * L * jt; t += gridDim.x) {
    const int bi = t / jt, j0 = (t - bi * jt) * 128 + 32 * wave;
    const int b = bi / L, i = bi - b * L;
    const int j = j0 + r;
    const bool live = j < L;
    const float* rij = p.r + (((size_t)b * L + i) * L + (live ? j : 0)) * C;
    const float* rji = p.r + (((size_t)b * L + (live ? j : 0)) * L + i) * C;
    f32x16 d[NBB];
#pragma unroll
    for (int bb = 0; bb < NBB; bb++)
#pragma unroll
      for (int e = 0; e < 16; e++) d[bb][e] = 0.f;
#pragma unroll
    for (int ks = 0; ks < C / 16; ks++) {
      const int c0 = 16 * ks + 8 * h;
      half8 s;
#pragma unroll
      for (int hh = 0; hh < 2; hh++) {
        const f32x4 x = *reinterpret_cast<const f32x4*>(rij + c0 + 4 * hh);
        const f32x4 y = *reinterpret_cast<const f32x4*>(rji + c0 + 4 * hh);
#pragma unroll
        for (int e = 0; e < 4; e++) s[4 * hh + e] = (half_t)(x[e] + y[e]);
      }
#pragma unroll
      for (int bb = 0; bb < NBB; bb++) d[bb] = mfma32(wa[bb][ks], s, d[bb]);
    }
    float mx = -INFINITY;
#pragma unroll
    for (int bb = 0; bb < NBB; bb++)
#pragma unroll
      for (int e = 0; e < 16; e++) {
        d[bb][e] += bias_s[32 * bb + acc_row32(e, lane)];
        mx = fmaxf(mx, d[bb][e]);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    float se = 0.f, sc = 0.f;
#pragma unroll
    for (int bb = 0; bb < NBB; bb++)
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const float ex = __expf(d[bb][e] - mx);
        se += ex;
        sc += ex * cent_s[32 * bb + acc_row32(e, lane)];
      }
    se += __shfl_xor(se, 32);
    sc += __shfl_xor(sc, 32);
    if (live && h == 0) p.ed[((size_t)b * L + i) * L + j] = sc / se;
  }
}

// ---- quantile of |x - y| ----------------------------------------------------------------------
// One workgroup of QT threads. Radix selection on the bit patterns of the non-negative values
// (their order is the value order): 3 passes of 11, 11 and 10 bits, each a histogram of the
// candidates still matching the selected high bits, for the two ranks that bracket the
// quantile at once; then linear interpolation between the two order statistics (the
// definition of torch.quantile). While both ranks share their selected high bits (always in
// the first pass, and in most later ones since the ranks are adjacent) one histogram serves
// both. Up to QT * QC values the patterns stay in registers after the first pass (thread tid
// holds values tid + QT j), so only one pass reads memory; beyond that every pass scans x and
// y in chunks of QT * QU values. Loads go through range-checked buffer descriptors with no
// branch around them, so a thread's loads are in flight together.
constexpr int QT = 1024;
__global__ __launch_bounds__(QT) void abs_diff_quantile_kernel(const float* __restrict__ x,
                                                               const float* __restrict__ y, size_t n, float q,
                                                               float* __restrict__ out) {
  constexpr int NBIN = 2048, BPT = NBIN / QT, NWV = QT / 64, QU = 8, QC = 56;
  constexpr uint32_t kNone = 0xffffffffu;  // an index past n: no prefix of a |value| matches it
  __shared__ uint32_t hist[2][NBIN];
  __shared__ uint32_t sel[2];
  __shared__ uint32_t wsum[2][NWV];
  __shared__ unsigned long long rank_s[2];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const double pos = (double)q * (double)(n - 1);
  const unsigned long long lo = (unsigned long long)pos;
  const unsigned long long hi = lo + 1 < n ? lo + 1 : lo;
  const float frac = (float)(pos - (double)lo);
  if (tid == 0) {
    rank_s[0] = lo;
    rank_s[1] = hi;
  }
  // Values [c0, c0 + cnt): x and y descriptors of exactly that range (y absent: range 0,
  // which loads zeros).
  auto chunk = [&](size_t c0, size_t cnt, rsrc_t& rx, rsrc_t& ry) {
    rx = make_rsrc_n(x + c0, (uint32_t)(cnt * 4));
    ry = make_rsrc_n(y ? y + c0 : x, y ? (uint32_t)(cnt * 4) : 0u);
  };
  // value tid + QT j: the per-thread part in the vector offset, the per-load part in the
  // scalar offset (no address register per load)
  auto ld = [&](const rsrc_t& r, int j) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, tid * 4, QT * 4 * j, 0);
  };
  // |x - y| as a bit pattern; an OR rather than a select, which would let the compiler sink
  // the loads under a branch
  auto pattern = [&](uint32_t xb, uint32_t yb, uint32_t i, size_t cnt) {
    return __float_as_uint(fabsf(__uint_as_float(xb) - __uint_as_float(yb))) | (i < cnt ? 0u : kNone);
  };
  const bool cached = n <= (size_t)QT * QC;
  uint32_t uc[QC];
  uint32_t prefix[2] = {0u, 0u}, mask = 0u;
  const int shifts[3] = {21, 10, 0}, widths[3] = {11, 11, 10};
#pragma unroll
  for (int ps = 0; ps < 3; ps++) {
    const int sh = shifts[ps];
    const uint32_t bmask = (1u << widths[ps]) - 1u;
    const bool shared = prefix[0] == prefix[1];  // block-uniform
    auto count = [&](uint32_t u) {
      const uint32_t bin = (u >> sh) & bmask;
      if ((u & mask) == prefix[0] && u != kNone) atomicAdd(&hist[0][bin], 1u);
      if (!shared && (u & mask) == prefix[1] && u != kNone) atomicAdd(&hist[1][bin], 1u);
    };
    for (int k = tid; k < 2 * NBIN; k += QT) (&hist[0][0])[k] = 0u;
    __syncthreads();
    if (cached) {
      if (ps == 0) {
        // all of x in flight, then y in groups of 8
        rsrc_t rx, ry;
        chunk(0, n, rx, ry);
#pragma unroll
        for (int j = 0; j < QC; j++) uc[j] = ld(rx, j);
#pragma unroll
        for (int g = 0; g < QC / 8; g++) {
          uint32_t yb[8];
#pragma unroll
          for (int j = 0; j < 8; j++) yb[j] = ld(ry, 8 * g + j);
#pragma unroll
          for (int j = 0; j < 8; j++)
            uc[8 * g + j] = pattern(uc[8 * g + j], yb[j], (uint32_t)(tid + QT * (8 * g + j)), n);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
#pragma unroll
      for (int j = 0; j < QC; j++) count(uc[j]);
    } else {
      for (size_t c0 = 0; c0 < n; c0 += (size_t)QT * QU) {
        const size_t cnt = n - c0 < (size_t)QT * QU ? n - c0 : (size_t)QT * QU;
        rsrc_t rx, ry;
        chunk(c0, cnt, rx, ry);
        uint32_t xb[QU], yb[QU];
#pragma unroll
        for (int j = 0; j < QU; j++) {
          xb[j] = ld(rx, j);
          yb[j] = ld(ry, j);
        }
#pragma unroll
        for (int j = 0; j < QU; j++) count(pattern(xb[j], yb[j], (uint32_t)(tid + QT * j), cnt));
      }
    }
    __syncthreads();
    // Each rank's bin: thread tid owns bins BPT tid .. BPT tid + BPT - 1; an exclusive scan of
    // the bin counts over the workgroup (64-lane scans, then the wave totals) gives each thread
    // the number of candidates below its bins, and the thread whose bins hold the rank records
    // the bin and the rank within it.
    {
      unsigned long long rk[2];
      uint32_t cb[2][BPT], c[2], inc[2];
#pragma unroll
      for (int t = 0; t < 2; t++) {
        const uint32_t* ht = hist[shared ? 0 : t];
        rk[t] = rank_s[t];
        c[t] = 0;
#pragma unroll
        for (int k = 0; k < BPT; k++) {
          cb[t][k] = ht[BPT * tid + k];
          c[t] += cb[t][k];
        }
        inc[t] = c[t];
      }
      for (int off = 1; off < 64; off <<= 1) {
#pragma unroll
        for (int t = 0; t < 2; t++) {
          const uint32_t o = __shfl_up(inc[t], off);
          if (lane >= off) inc[t] += o;
        }
      }
      if (lane == 63) {
        wsum[0][wv] = inc[0];
        wsum[1][wv] = inc[1];
      }
      __syncthreads();
#pragma unroll
      for (int t = 0; t < 2; t++) {
        unsigned long long before = inc[t] - c[t];
        for (int w = 0; w < wv; w++) before += wsum[t][w];
        if (rk[t] >= before && rk[t] < before + c[t]) {  // exactly one thread
          int k = 0;
          while (k < BPT - 1 && rk[t] >= before + cb[t][k]) before += cb[t][k++];
          sel[t] = (uint32_t)(BPT * tid + k);
          rank_s[t] = rk[t] - before;
        }
      }
    }
    __syncthreads();
    prefix[0] |= sel[0] << sh;
    prefix[1] |= sel[1] << sh;
    mask |= bmask << sh;
    __syncthreads();
  }
  if (tid == 0) {
    const float a = __uint_as_float(prefix[0]), b = __uint_as_float(prefix[1]);
    out[0] = a + frac * (b - a);
  }
}

hipError_t launch_parcae_step(const ParcaeArgs& a, int grid, hipStream_t s) {
  hipLaunchKernelGGL(parcae_step_kernel, dim3(grid), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_expected_distance(const DistoArgs& a, int grid, hipStream_t s) {
  if (a.nbins == 64)
    hipLaunchKernelGGL(expected_distance_kernel<2>, dim3(grid), dim3(256), 0, s, a);
  else if (a.nbins == 128)
    hipLaunchKernelGGL(expected_distance_kernel<4>, dim3(grid), dim3(256), 0, s, a);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_abs_diff_quantile(const float* x, const float* y, size_t n, float q, float* out, hipStream_t s) {
  hipLaunchKernelGGL(abs_diff_quantile_kernel, dim3(1), dim3(QT), 0, s, x, y, n, q, out);
  return hipGetLastError();
}

}  // namespace esm
