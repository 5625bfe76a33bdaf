// Kernels of the recycling step around the trunk (var_6b_mlx_loop.py:67-85,
// var_adaptive_loops.py:41-46, :109-118):
//   parcae_step          z <- a * z + LN(z_init + refined) @ B^T on every cell (fp32 state)
//   expected_distance    softmax((r + r^T) @ W^T + b) . centres per pair (distogram head)
//   abs_diff_quantile    the q-th quantile (linear interpolation) of |x - y| (exit signal)
// C = 128 or 256 pair channels (a template parameter of the first two).
#include "common.h"
#include "kernels.h"

namespace esm {

// ---- parcae step ----------------------------------------------------------------------------
// Persistent, 4 waves per workgroup; a tile is 32 consecutive cells. Wave w owns output
// channels [w CC/4, (w+1) CC/4) (OB = CC/128 blocks of 32) and keeps those rows of B (fp16) as
// MFMA A fragments. Per tile: u = z_init + refined, LayerNorm (16 lanes per cell, lane l
// holding the 8-channel chunks l + 16 t, fp32 statistics) into LDS as fp16, one barrier,
// D[co][cell] = B[co][:] . LN(u)[cell][:] (fp32 accumulation), then a[co] * z + D in fp32,
// 16-byte stores (4 consecutive channels per lane and quad).
template <int CC>
__global__ __launch_bounds__(256, 1) void parcae_step_kernel(ParcaeArgs p) {
  constexpr int OB = CC / 128;       // 32-channel output blocks per wave
  constexpr int NCH = CC / 128;      // 8-channel chunks per lane in the LayerNorm
  constexpr int NSTR = CC + 8;       // LDS row stride (halfs) of the LayerNormed tile
  __shared__ __align__(16) half_t n_s[32 * NSTR];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 31, h = lane >> 5;
  half8 bw[OB][CC / 16];
#pragma unroll
  for (int ob = 0; ob < OB; ob++) {
    const half_t* row = p.b_mat + (size_t)(wave * (CC / 4) + 32 * ob + r) * CC;
#pragma unroll
    for (int ks = 0; ks < CC / 16; ks++) bw[ob][ks] = ld16(row + 16 * ks + 8 * h);
  }
  const int l16 = lane & 15;
  float g[NCH][8], bb[NCH][8];
#pragma unroll
  for (int t = 0; t < NCH; t++)
#pragma unroll
    for (int e = 0; e < 8; e++) {
      g[t][e] = p.ln_w[8 * (l16 + 16 * t) + e];
      bb[t][e] = p.ln_b[8 * (l16 + 16 * t) + e];
    }
  float av[OB][16];  // a for this lane's output channels
#pragma unroll
  for (int ob = 0; ob < OB; ob++)
#pragma unroll
    for (int i = 0; i < 16; i++) av[ob][i] = p.a[wave * (CC / 4) + 32 * ob + acc_row32(i, lane)];

  const rsrc_t rz = make_rsrc(p.z), ri = make_rsrc(p.z_init), rr = make_rsrc(p.refined), ro = make_rsrc(p.z_out);
  const size_t ncells = p.ncells;
  for (int tile = blockIdx.x; tile < p.ntiles; tile += gridDim.x) {
    const size_t cell0 = (size_t)tile * 32;
    // 1. u -> LayerNorm -> LDS
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int cl = (tid >> 4) + 16 * i;
      const bool live = cell0 + cl < ncells;
      float v[NCH][8];
#pragma unroll
      for (int t = 0; t < NCH; t++) {
        const uint32_t off = live ? (uint32_t)(((cell0 + cl) * CC + 8 * (l16 + 16 * t)) * 4u) : kOOB;
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
          const f32x4 a4 = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(ri, (int)(off + 16u * hh), 0, 0));
          const f32x4 b4 = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rr, (int)(off + 16u * hh), 0, 0));
#pragma unroll
          for (int e = 0; e < 4; e++) v[t][4 * hh + e] = a4[e] + b4[e];
        }
      }
      float s = 0.f;
#pragma unroll
      for (int t = 0; t < NCH; t++)
#pragma unroll
        for (int e = 0; e < 8; e++) s += v[t][e];
      const float mean = row16_sum(s) * (1.0f / CC);
      float q = 0.f;
#pragma unroll
      for (int t = 0; t < NCH; t++)
#pragma unroll
        for (int e = 0; e < 8; e++) {
          v[t][e] -= mean;
          q += v[t][e] * v[t][e];
        }
      const float rstd = rsqrtf(row16_sum(q) * (1.0f / CC) + p.eps);
#pragma unroll
      for (int t = 0; t < NCH; t++) {
        half8 o;
#pragma unroll
        for (int e = 0; e < 8; e++) o[e] = (half_t)(v[t][e] * rstd * g[t][e] + bb[t][e]);
        st16(&n_s[cl * NSTR + 8 * (l16 + 16 * t)], o);
      }
    }
    __syncthreads();
    // 2. D[co][cell] over the wave's output channels
    f32x16 d[OB];
#pragma unroll
    for (int ob = 0; ob < OB; ob++)
#pragma unroll
      for (int i = 0; i < 16; i++) d[ob][i] = 0.f;
#pragma unroll
    for (int ks = 0; ks < CC / 16; ks++) {
      const half8 nb = ld16(&n_s[r * NSTR + 16 * ks + 8 * h]);
#pragma unroll
      for (int ob = 0; ob < OB; ob++) d[ob] = mfma32(bw[ob][ks], nb, d[ob]);
    }
    // 3. a * z + D for the lane's cell and 4 quads of 4 consecutive channels per block
    const bool live = cell0 + r < ncells;
#pragma unroll
    for (int ob = 0; ob < OB; ob++)
#pragma unroll
      for (int r4 = 0; r4 < 4; r4++) {
        const int co = wave * (CC / 4) + 32 * ob + acc_row32(4 * r4, lane);
        const uint32_t off = live ? (uint32_t)(((cell0 + r) * CC + co) * 4u) : kOOB;
        const f32x4 z4 = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rz, (int)off, 0, 0));
        f32x4 o;
#pragma unroll
        for (int e = 0; e < 4; e++) o[e] = av[ob][4 * r4 + e] * z4[e] + d[ob][4 * r4 + e];
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o), ro, (int)off, 0, 0);
      }
    __syncthreads();  // n_s is rewritten by the next tile
  }
}

// ---- expected distance ----------------------------------------------------------------------
// The head is symmetric in (i, j): s[i,j] = r[i,j] + r[j,i] is the same fp32 sum both ways
// round, so only pairs j >= i are computed and each result is written to ed[i,j] and ed[j,i];
// every cell of r is then read from HBM once (both orders per pair: r[i,j] and r[j,i]).
// One wave per 32 pairs (b, i, j0 .. j0+31) with j0 = 32 * jt over the tiles jt >= i / 32;
// lanes for j < i (the diagonal tile) re-read the cell (i, i) and write nothing. Waves take
// units independently (no workgroup barrier after the set-up).
// Loads: each instruction reads whole cells (64 lanes x 16 bytes = 256 / CC cells), r[i,j]
// and r[j,i] in the same lane layout, so the fp32 sum is formed in registers, rounded to fp16
// and stored to the wave's LDS rows s[cell][c]. The MFMA's B operand (column = pair, k =
// channel) is read from there; A = the head's weight rows (bins), held in registers, or for
// the widest heads (128 bins at 256 channels: 256 registers of fragments) read from an LDS
// copy per k-step. A lane then holds its pair's logits for 16 bins per 32-bin block: the
// softmax over bins is a register reduction plus one exchange between the lane halves.
// Bias and centres come from LDS.
template <int NBB, int CC>  // 32-bin blocks, channels
__global__ __launch_bounds__(256, 1) void expected_distance_kernel(DistoArgs p) {
  constexpr int NB = 32 * NBB;
  constexpr bool WLDS = NBB * CC > 512;   // fragments from LDS instead of registers
  constexpr int WS = CC + 8;              // LDS row stride (halfs) of the weight copy and the pair rows
  constexpr int LPC = CC / 4;             // lanes per cell in a load instruction
  constexpr int CPI = 64 / LPC;           // cells per load instruction
  constexpr int QB = CC == 128 ? 16 : 8;  // load instructions in flight per array
  __shared__ float bias_s[NB], cent_s[NB];
  __shared__ __align__(16) half_t w_s[WLDS ? NB * WS : 8];
  __shared__ __align__(16) half_t s_s[4][32 * WS];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 31, h = lane >> 5;
  for (int k = tid; k < NB; k += 256) {
    bias_s[k] = p.bias[k];
    cent_s[k] = p.centers[k];
  }
  half8 wa[WLDS ? 1 : NBB][WLDS ? 1 : CC / 16];
  if constexpr (WLDS) {
    for (int q = tid; q < NB * (CC / 8); q += 256) {
      const int row = q / (CC / 8), j = q - row * (CC / 8);
      st16(&w_s[row * WS + 8 * j], ld16(p.w + (size_t)row * CC + 8 * j));
    }
  } else {
#pragma unroll
    for (int bb = 0; bb < NBB; bb++)
#pragma unroll
      for (int ks = 0; ks < CC / 16; ks++) wa[bb][ks] = ld16(p.w + (size_t)(32 * bb + r) * CC + 16 * ks + 8 * h);
  }
  __syncthreads();

  half_t* sw = s_s[wave];
  const int L = p.L;
  const int JT = (L + 31) / 32;  // 32-pair tiles per row
  // units per batch: rows of block I (32 rows, the last one L - 32 I) hold JT - I tiles each
  int per_b = 0;
  for (int I = 0; I < JT; I++) per_b += min(32, L - 32 * I) * (JT - I);
  const int U = p.B * per_b;
  const int lc = lane / LPC, f = 4 * (lane - lc * LPC);  // cell within an instruction, channel
  for (int u = blockIdx.x * 4 + wave; u < U; u += gridDim.x * 4) {
    const int b = u / per_b;
    int rem = u - b * per_b, I = 0;
    while (rem >= 32 * (JT - I)) {
      rem -= 32 * (JT - I);
      I++;
    }
    const int row = rem / (JT - I), jt = I + (rem - row * (JT - I));
    const int i = 32 * I + row;
    const float* ri = p.r + ((size_t)b * L + i) * L * CC;  // row i
    const float* rc = p.r + (size_t)b * L * L * CC + (size_t)i * CC;  // column i
#pragma unroll
    for (int q0 = 0; q0 < 32 / CPI; q0 += QB) {
      f32x4 x[QB], y[QB];
#pragma unroll
      for (int q = 0; q < QB; q++) {
        const int j = 32 * jt + CPI * (q0 + q) + lc;
        const int jj = j >= i && j < L ? j : i;
        x[q] = *reinterpret_cast<const f32x4*>(ri + (size_t)jj * CC + f);
        y[q] = *reinterpret_cast<const f32x4*>(rc + (size_t)jj * L * CC + f);
      }
#pragma unroll
      for (int q = 0; q < QB; q++) {
        half4 v;
#pragma unroll
        for (int e = 0; e < 4; e++) v[e] = (half_t)(x[q][e] + y[q][e]);
        *reinterpret_cast<half4*>(&sw[(CPI * (q0 + q) + lc) * WS + f]) = v;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    f32x16 d[NBB];
#pragma unroll
    for (int bb = 0; bb < NBB; bb++)
#pragma unroll
      for (int e = 0; e < 16; e++) d[bb][e] = 0.f;
#pragma unroll
    for (int ks = 0; ks < CC / 16; ks++) {
      const int c0 = 16 * ks + 8 * h;
      const half8 sv = ld16(&sw[r * WS + c0]);
#pragma unroll
      for (int bb = 0; bb < NBB; bb++) {
        const half8 w = WLDS ? ld16(&w_s[(32 * bb + r) * WS + c0]) : wa[WLDS ? 0 : bb][WLDS ? 0 : ks];
        d[bb] = mfma32(w, sv, d[bb]);
      }
    }
    // the next unit's stores to sw come after every lane's fragment reads
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
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
    const int j = 32 * jt + r;
    if (j >= i && j < L && h == 0) {
      const float v = sc / se;
      p.ed[((size_t)b * L + i) * L + j] = v;
      if (j != i) p.ed[((size_t)b * L + j) * L + i] = v;
    }
  }
}

// ---- quantile of |x - y| ----------------------------------------------------------------------
// Beyond the register-held sizes (abs_diff_quantile_regs_kernel below): one workgroup of QT
// threads. Radix selection on the bit patterns of the non-negative values (their order is the
// value order): 3 passes of 11, 11 and 10 bits, each a histogram of the candidates still
// matching the selected high bits, for the two ranks that bracket the quantile at once; then
// linear interpolation between the two order statistics (the definition of torch.quantile).
// While both ranks share their selected high bits (always in the first pass, and in most later
// ones since the ranks are adjacent) one histogram serves both. Every pass scans x and y in
// chunks of QT * QU values through range-checked buffer descriptors with no branch around the
// loads, so a thread's loads are in flight together.
constexpr int QT = 1024;
__global__ __launch_bounds__(QT) void abs_diff_quantile_kernel(const float* __restrict__ x,
                                                               const float* __restrict__ y, size_t n, float q,
                                                               float* __restrict__ out) {
  constexpr int NBIN = 2048, BPT = NBIN / QT, NWV = QT / 64, QU = 8;
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

// Up to QR * QCR = 57,344 values (every pair grid up to L = 239): the same order statistics in
// two passes, the values held in registers (1024 threads of 56 values: sixteen waves hide the
// scans' and the atomics' latency better than eight of 112, 17.6 against 21.5 us at L = 238,
// within the 128 registers a thread has at that size). Pass 0 counts the 15 bits
// under the (zero) sign bit, bits 30..16, in 32,768 bins (128 KB of LDS); a workgroup-wide scan
// gives the bins b0, b1 of the two ranks. When b0 == b1 (nearly always: the ranks are adjacent)
// pass 1 counts the low 16 bits of that bin's values in 65,536 bins of 16-bit counters packed two
// to a word (no count can exceed n < 2^16), and a second scan gives both ranks' low bits. When
// b0 != b1 the lower rank is the largest value of b0 and the upper the smallest of b1: one
// maximum and one minimum, reduced per wave before a single LDS atomic each.
constexpr int QR = 1024, QCR = 56;
__global__ __launch_bounds__(QR) void abs_diff_quantile_regs_kernel(const float* __restrict__ x,
                                                                    const float* __restrict__ y, uint32_t n,
                                                                    float q, float* __restrict__ out) {
  constexpr int NWV = QR / 64;
  constexpr int NW0 = 1 << 15;             // words of the histogram: pass-0 bins, or pass 1's packed pairs
  constexpr int WPT = NW0 / QR;            // words per thread in the scans
  constexpr int CPT = WPT / 4;             // their 16-byte chunks
  constexpr uint32_t kNone = 0xffffffffu;  // past n: its top bits (0xffff) match no bin
  static_assert((CPT & (CPT - 1)) == 0 && QCR % 8 == 0, "a power-of-two chunk count; y in groups of 8");
  __shared__ __align__(16) uint32_t h[NW0];
  __shared__ uint32_t wsum[NWV];
  __shared__ uint32_t sel[2], rk_s[2], mm[2];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const double pos = (double)q * (double)(n - 1);
  const uint32_t lo = (uint32_t)pos, hi = lo + 1 < n ? lo + 1 : lo;
  const float frac = (float)(pos - (double)lo);
  const int nj = (int)(4 * ((n / 4 + QR - 1) / QR));  // slots j < nj can hold values of the pieces

  auto zero_hist = [&]() {  // one address register stepped through (unrolled, the offsets past 64 KB each need one)
#pragma unroll 1
    for (int k = tid; k < NW0 / 4; k += QR) reinterpret_cast<uint4*>(h)[k] = make_uint4(0u, 0u, 0u, 0u);
  };
  // Both ranks' bins in the histogram h (PK: two 16-bit counts per word, the even bin low).
  // Thread tid owns words WPT tid .. WPT tid + WPT - 1; it sums them in a lane-rotated order (of
  // 16-byte chunks: the 8 lanes one read serves hit 8 distinct 4-bank groups), a workgroup scan
  // of the sums gives the counts before each thread's words, and the thread whose words hold a
  // rank finds the chunk, then the word and the bin. sel[t] = the bin, rk_s[t] = the rank within it.
  auto select = [&](auto packed, uint32_t r0, uint32_t r1) {
    constexpr bool PK = decltype(packed)::value;
    auto wcount = [](uint32_t w) { return PK ? (w & 0xffffu) + (w >> 16) : w; };
    uint32_t c = 0;
#pragma unroll
    for (int k = 0; k < CPT; k++) {
      const uint4 w = *reinterpret_cast<const uint4*>(&h[WPT * tid + 4 * ((k + lane) & (CPT - 1))]);
      c += wcount(w.x) + wcount(w.y) + wcount(w.z) + wcount(w.w);
    }
    uint32_t inc = c;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const uint32_t o = __shfl_up(inc, off);
      if (lane >= off) inc += o;
    }
    if (lane == 63) wsum[wv] = inc;
    __syncthreads();
    uint32_t before = inc - c;
    for (int w = 0; w < wv; w++) before += wsum[w];
#pragma unroll
    for (int t = 0; t < 2; t++) {
      const uint32_t r = t ? r1 : r0;
      if (r >= before && r < before + c) {  // exactly one thread per rank
        uint4 ch[CPT];  // all of the thread's chunks in flight
#pragma unroll
        for (int k = 0; k < CPT; k++) ch[k] = *reinterpret_cast<const uint4*>(&h[WPT * tid + 4 * k]);
        uint32_t acc = before;
        int kc = CPT - 1;
#pragma unroll
        for (int k = 0; k < CPT - 1; k++) {
          const uint32_t cs = wcount(ch[k].x) + wcount(ch[k].y) + wcount(ch[k].z) + wcount(ch[k].w);
          if (kc == CPT - 1) {
            if (r < acc + cs)
              kc = k;
            else
              acc += cs;
          }
        }
        uint4 cw = ch[0];
#pragma unroll
        for (int k = 1; k < CPT; k++)
          if (kc == k) cw = ch[k];
        const uint32_t wd[4] = {cw.x, cw.y, cw.z, cw.w};
        int bin = -1;
#pragma unroll
        for (int k = 0; k < 4; k++)
#pragma unroll
          for (int e = 0; e < (PK ? 2 : 1); e++) {
            const uint32_t cnt = PK ? (e ? wd[k] >> 16 : wd[k] & 0xffffu) : wd[k];
            if (bin < 0) {
              if (r < acc + cnt)
                bin = (PK ? 2 : 1) * (WPT * tid + 4 * kc + k) + e;
              else
                acc += cnt;
            }
          }
        sel[t] = (uint32_t)bin;
        rk_s[t] = r - acc;
      }
    }
    __syncthreads();
  };

  zero_hist();
  // Loads as 16-byte pieces (a quarter of the load instructions: their issue, not the bytes,
  // bounds a single workgroup's reads): thread tid holds values 4 (tid + QR j) .. +3, j < QCR / 4,
  // of the first n4 = n - n % 4 (every piece wholly inside or wholly past that range), and
  // threads 0 .. n % 4 - 1 hold the tail value n4 + tid in ut (kNone elsewhere). All of x in
  // flight, then y two pieces at a time; range-checked descriptors, no branch around the loads.
  uint32_t uc[QCR], ut;
  {
    const uint32_t n4 = n & ~3u;
    const rsrc_t rx = make_rsrc_n(x, n4 * 4u), ry = make_rsrc_n(y ? y : x, y ? n4 * 4u : 0u);
#pragma unroll
    for (int j = 0; j < QCR / 4; j++) {
      const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, tid * 16, QR * 16 * j, 0));
#pragma unroll
      for (int e = 0; e < 4; e++) uc[4 * j + e] = v[e];
    }
#pragma unroll
    for (int g = 0; g < QCR / 8; g++) {
      u32x4 yb[2];
#pragma unroll
      for (int h2 = 0; h2 < 2; h2++)
        yb[h2] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(ry, tid * 16, QR * 16 * (2 * g + h2), 0));
#pragma unroll
      for (int h2 = 0; h2 < 2; h2++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int j = 4 * (2 * g + h2) + e;
          const uint32_t i = 4u * (uint32_t)(tid + QR * (2 * g + h2)) + e;
          uc[j] = __float_as_uint(fabsf(__uint_as_float(uc[j]) - __uint_as_float(yb[h2][e]))) | (i < n4 ? 0u : kNone);
        }
      __builtin_amdgcn_sched_barrier(0);
    }
    const rsrc_t tx = make_rsrc_n(x, n * 4u), ty = make_rsrc_n(y ? y : x, y ? n * 4u : 0u);
    const bool tail = (uint32_t)tid < n - n4;
    const uint32_t toff = tail ? (n4 + (uint32_t)tid) * 4u : kOOB;
    const uint32_t xt = __builtin_amdgcn_raw_buffer_load_b32(tx, (int)toff, 0, 0);
    const uint32_t yt = __builtin_amdgcn_raw_buffer_load_b32(ty, (int)toff, 0, 0);
    ut = __float_as_uint(fabsf(__uint_as_float(xt) - __uint_as_float(yt))) | (tail ? 0u : kNone);
  }
  __syncthreads();  // the histogram is zero
#pragma unroll
  for (int j = 0; j < QCR; j++)
    if (j < nj && uc[j] != kNone) atomicAdd(&h[uc[j] >> 16], 1u);
  if (ut != kNone) atomicAdd(&h[ut >> 16], 1u);
  __syncthreads();
  select(std::false_type{}, lo, hi);
  const uint32_t b0 = sel[0], b1 = sel[1];
  uint32_t d0, d1;
  if (b0 == b1) {  // block-uniform
    const uint32_t r0 = rk_s[0], r1 = rk_s[1];
    __syncthreads();  // every thread has read sel and rk_s
    zero_hist();
    __syncthreads();
#pragma unroll
    for (int j = 0; j <= QCR; j++) {  // j == QCR: the tail value
      const uint32_t u = j < QCR ? uc[j] : ut;
      if ((j < nj || j == QCR) && (u >> 16) == b0) atomicAdd(&h[(u & 0xffffu) >> 1], 1u << ((u & 1u) << 4));
    }
    __syncthreads();
    select(std::true_type{}, r0, r1);
    d0 = sel[0];
    d1 = sel[1];
  } else {
    if (tid == 0) {
      mm[0] = 0u;
      mm[1] = 0xffffu;
    }
    uint32_t mx = 0u, mn = 0xffffu;
#pragma unroll
    for (int j = 0; j <= QCR; j++) {  // j == QCR: the tail value
      const uint32_t u = j < QCR ? uc[j] : ut;
      const bool on = j < nj || j == QCR;
      if (on && (u >> 16) == b0) mx = max(mx, u & 0xffffu);
      if (on && (u >> 16) == b1) mn = min(mn, u & 0xffffu);
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      mx = max(mx, (uint32_t)__shfl_xor((int)mx, off));
      mn = min(mn, (uint32_t)__shfl_xor((int)mn, off));
    }
    __syncthreads();  // mm initialised
    if (lane == 0) {
      atomicMax(&mm[0], mx);
      atomicMin(&mm[1], mn);
    }
    __syncthreads();
    d0 = mm[0];
    d1 = mm[1];
  }
  if (tid == 0) {
    const float a = __uint_as_float((b0 << 16) | d0), b = __uint_as_float((b1 << 16) | d1);
    out[0] = a + frac * (b - a);
  }
}

hipError_t launch_parcae_step(const ParcaeArgs& a, int grid, hipStream_t s) {
  if (a.C == 128)
    ESM_LAUNCH(parcae_step_kernel<128>, dim3(grid), dim3(256), 0, s, a);
  else if (a.C == 256)
    ESM_LAUNCH(parcae_step_kernel<256>, dim3(grid), dim3(256), 0, s, a);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_expected_distance(const DistoArgs& a, int grid, hipStream_t s) {
  if (a.nbins == 64 && a.C == 128)
    ESM_LAUNCH((expected_distance_kernel<2, 128>), dim3(grid), dim3(256), 0, s, a);
  else if (a.nbins == 128 && a.C == 128)
    ESM_LAUNCH((expected_distance_kernel<4, 128>), dim3(grid), dim3(256), 0, s, a);
  else if (a.nbins == 64 && a.C == 256)
    ESM_LAUNCH((expected_distance_kernel<2, 256>), dim3(grid), dim3(256), 0, s, a);
  else if (a.nbins == 128 && a.C == 256)
    ESM_LAUNCH((expected_distance_kernel<4, 256>), dim3(grid), dim3(256), 0, s, a);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_abs_diff_quantile(const float* x, const float* y, size_t n, float q, float* out, hipStream_t s) {
  if (n <= (size_t)QR * QCR)
    ESM_LAUNCH(abs_diff_quantile_regs_kernel, dim3(1), dim3(QR), 0, s, x, y, (uint32_t)n, q, out);
  else
    ESM_LAUNCH(abs_diff_quantile_kernel, dim3(1), dim3(QT), 0, s, x, y, n, q, out);
  return hipGetLastError();
}

}  // namespace esm
