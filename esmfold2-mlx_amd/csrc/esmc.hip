// Kernels of the ESMC transformer block around the 8-bit linear (mlx_esmc.py:84-102),
// other than the q8 GEMMs themselves (q8.hip):
//   esmc_ln        x' = x + alpha*y (fp32 residual, optional; y fp16 or the q8 linear's
//                  fp32 split partials), h = LN(x') -> fp16 or fp32
//   esmc_qk_rope   QK-LayerNorm over the full width (weight only, fp32 statistics),
//                  NeoX rotary embedding, head-major q, k, v for the attention
//   esmc_attention softmax(q k^T * scale, same-chain mask) v, 32 queries of one head
//                  per workgroup, keys split over its 4 waves, MFMA for both products
//   esmc_swiglu    silu(x1) * x2 in fp32, one rounding
// Row kernels run one 256-thread workgroup per token row (the rows are a few KB: these
// are launch- and latency-bound, a few microseconds each at 238 tokens).
#include "common.h"
#include "kernels.h"

namespace esm {

namespace {
constexpr int NTR = 256;  // threads of the row kernels
}

// Sum over the workgroup (4 waves): DPP within rows of 16, a cross-row butterfly, LDS across waves.
DEV float wg_sum(float v, float* red) {
  v = row16_sum(v);
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  const int w = threadIdx.x >> 6;
  __syncthreads();  // red is reused by consecutive calls
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

typedef float float2v __attribute__((ext_vector_type(2)));
// Two sums over the workgroup at once (one pair of barriers).
DEV float2v wg_sum2(float a, float b, float (*red)[4]) {
  a = row16_sum(a);
  b = row16_sum(b);
  a += __shfl_xor(a, 16);
  b += __shfl_xor(b, 16);
  a += __shfl_xor(a, 32);
  b += __shfl_xor(b, 32);
  const int w = threadIdx.x >> 6;
  __syncthreads();  // red is reused by consecutive calls
  if ((threadIdx.x & 63) == 0) {
    red[0][w] = a;
    red[1][w] = b;
  }
  __syncthreads();
  return float2v{red[0][0] + red[0][1] + red[0][2] + red[0][3], red[1][0] + red[1][1] + red[1][2] + red[1][3]};
}

// ---- residual + LayerNorm -------------------------------------------------------------------
// Thread t holds the element groups i = 4 (t + 256 j), j < NJ = ceil(D / 1024). Every load is
// a range-checked buffer load (groups past D load zeros and are masked out of the sums) issued
// before the first use, and the split count of the common plans is a template parameter, so
// a row's x and all of its split partials are in flight together: with a branch around each
// group and a loop over the splits every partial waited for the one before it. The sums keep
// their order (splits in order, rounded once to fp16, then the residual; groups in order for
// the statistics).
template <int NJ, int NSPL>  // NSPL: y's split partials, a fixed count (unrolled) or -1 (any count)
__global__ __launch_bounds__(NTR) void esmc_ln_kernel(EsmcLnArgs p) {
  __shared__ float red[4];
  const int row = blockIdx.x, D = p.D, t = threadIdx.x;
  const uint32_t rowb = (uint32_t)D * 4u;
  auto off = [&](int j) { return (uint32_t)(4 * (t + NTR * j)) * 4u; };  // bytes into an fp32 row
  auto valid = [&](int j) { return 4 * (t + NTR * j) < D; };
  auto ld4 = [&](rsrc_t r, int j) { return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off(j), 0, 0)); };
  const rsrc_t rx = make_rsrc_n(p.x + (size_t)row * D, rowb);
  f32x4 v[NJ];
#pragma unroll
  for (int j = 0; j < NJ; j++) v[j] = ld4(rx, j);
  const bool res = p.y || p.yp;
  if (p.yp) {
    const size_t plane = (size_t)p.M * D;
    auto part = [&](int sp) { return make_rsrc_n(p.yp + sp * plane + (size_t)row * D, rowb); };
    f32x4 a[NJ];
    if constexpr (NSPL > 0) {  // every partial in flight at once
      f32x4 l[NSPL][NJ];
#pragma unroll
      for (int sp = 0; sp < NSPL; sp++)
#pragma unroll
        for (int j = 0; j < NJ; j++) l[sp][j] = ld4(part(sp), j);
#pragma unroll
      for (int j = 0; j < NJ; j++) {
        a[j] = l[0][j];
#pragma unroll
        for (int sp = 1; sp < NSPL; sp++) a[j] += l[sp][j];
      }
    } else {  // any count: one split's groups in flight at a time
#pragma unroll
      for (int j = 0; j < NJ; j++) a[j] = ld4(part(0), j);
      for (int sp = 1; sp < p.splits; sp++)
#pragma unroll
        for (int j = 0; j < NJ; j++) a[j] += ld4(part(sp), j);
    }
#pragma unroll
    for (int j = 0; j < NJ; j++)
#pragma unroll
      for (int e = 0; e < 4; e++) v[j][e] += p.alpha * (float)(half_t)a[j][e];
  } else if (p.y) {
    const rsrc_t ry = make_rsrc_n(p.y + (size_t)row * D, (uint32_t)D * 2u);
#pragma unroll
    for (int j = 0; j < NJ; j++) {
      const half4 yy = __builtin_bit_cast(half4, __builtin_amdgcn_raw_buffer_load_b64(ry, (int)(off(j) / 2), 0, 0));
#pragma unroll
      for (int e = 0; e < 4; e++) v[j][e] += p.alpha * (float)yy[e];
    }
  }
  const rsrc_t rxo = make_rsrc_n(p.x_out + (size_t)row * D, res ? rowb : 0u);
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    if (res) __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v[j]), rxo, (int)off(j), 0, 0);
    const float sj = s + (v[j][0] + v[j][1] + v[j][2] + v[j][3]);
    s = valid(j) ? sj : s;
  }
  const float mean = wg_sum(s, red) / D;
  float q = 0.f;
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    float qj = q;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      v[j][e] -= mean;
      qj += v[j][e] * v[j][e];
    }
    q = valid(j) ? qj : q;
  }
  const float rstd = rsqrtf(wg_sum(q, red) / D + p.eps);
  const rsrc_t rw = make_rsrc_n(p.w, rowb), rb = make_rsrc_n(p.b ? (const void*)p.b : (const void*)p.w, p.b ? rowb : 0u);
  const rsrc_t rh = make_rsrc_n(p.h ? (void*)(p.h + (size_t)row * D) : (void*)p.w, p.h ? (uint32_t)D * 2u : 0u);
  const rsrc_t rh32 = make_rsrc_n(p.h32 ? (void*)(p.h32 + (size_t)row * D) : (void*)p.w, p.h32 ? rowb : 0u);
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    const f32x4 w4 = ld4(rw, j), b4 = ld4(rb, j);  // (no bias: zeros)
    f32x4 o;
#pragma unroll
    for (int e = 0; e < 4; e++) o[e] = v[j][e] * rstd * w4[e] + b4[e];
    if (p.h) bstore8(rh, off(j) / 2, half4{(half_t)o[0], (half_t)o[1], (half_t)o[2], (half_t)o[3]});
    if (p.h32) __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o), rh32, (int)off(j), 0, 0);
  }
}

// ---- QK-LayerNorm + RoPE, head-major outputs ---------------------------------------------------
// One thread per chunk of 8 rotation pairs: chunk u < D/16 of q, else of k (u' = u mod D/16);
// pairs (e, e + 32) of head u' / 4 at e = 8 (u' % 4) .. + 7, so a chunk is two 16-byte loads
// and two 16-byte stores; thread t also moves v's 8 halfs at 8 t. The workgroup has
// roundup(D/8, 64) threads (the D/8 chunks of q and k; 320 at D = 2560, at most 512), so no
// wave carries a second chunk. Every load is issued first (v, the q/k chunk through a
// range-checked descriptor of the row, its LayerNorm weights) and v leaves as soon as it has
// arrived. The LayerNorm statistics of q and k are reduced together. The rotation's sines and
// cosines are taken before the reductions, from the angle in revolutions (the hardware sine
// of its fractional part; the angle itself is an fp32 product, as before): 5.4 -> 4.5 us at 238
// tokens against the precise library sincos.
constexpr int kRopeMaxThreads = 512;
DEV float2v wg_sum2_n(float a, float b, float (*red)[kRopeMaxThreads / 64]) {
  a = row16_sum(a);
  b = row16_sum(b);
  a += __shfl_xor(a, 16);
  b += __shfl_xor(b, 16);
  a += __shfl_xor(a, 32);
  b += __shfl_xor(b, 32);
  const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();  // red is reused by consecutive calls
  if ((threadIdx.x & 63) == 0) {
    red[0][w] = a;
    red[1][w] = b;
  }
  __syncthreads();
  float sa = red[0][0], sb = red[1][0];
  for (int k = 1; k < nw; k++) {
    sa += red[0][k];
    sb += red[1][k];
  }
  return float2v{sa, sb};
}

__global__ __launch_bounds__(kRopeMaxThreads) void esmc_qk_rope_kernel(EsmcRopeArgs p) {
  __shared__ float red[2][kRopeMaxThreads / 64];
  constexpr int HD = 64, HALF = 32;
  const int row = blockIdx.x, D = p.H * HD, nq = D / 16, t = threadIdx.x;
  const int b = row / p.L, l = row - b * p.L;
  const half_t* src = p.qkv + (size_t)row * 3 * D;
  const rsrc_t rs = make_rsrc_n(src, (uint32_t)(3 * D) * 2u);
  const int ev = 8 * t;
  const half8 vv = bload16(rs, ev < D ? (uint32_t)(2 * D + ev) * 2u : kOOB);
  const bool ok = t < 2 * nq;
  const int which = t >= nq, uu = t - which * nq, hh = uu >> 2, i0 = 8 * (uu & 3);
  const uint32_t off = (uint32_t)(which * D + hh * HD + i0) * 2u;
  const half8 x1 = bload16(rs, ok ? off : kOOB), x2 = bload16(rs, ok ? off + 2u * HALF : kOOB);
  const float* w = ok ? (which ? p.k_ln : p.q_ln) + hh * HD + i0 : p.q_ln;
  const f32x4 w0 = *reinterpret_cast<const f32x4*>(w), w1 = *reinterpret_cast<const f32x4*>(w + 4);
  const f32x4 w2 = *reinterpret_cast<const f32x4*>(w + HALF), w3 = *reinterpret_cast<const f32x4*>(w + HALF + 4);
  if (ev < D) st16(p.v + (((size_t)b * p.H + ev / HD) * p.L + l) * HD + ev % HD, vv);  // v: head-major

  // rotation of pair i = i0 + e at position l: the angle l * base^(-2i/64) in revolutions (its
  // fractional part), by the hardware sine and cosine; independent of the statistics, so it
  // runs under the reductions' barriers
  float sn[8], cs[8];
#pragma unroll
  for (int e = 0; e < 8; e++) {
    float rev = (float)l * (exp2f(-(float)(2 * (i0 + e)) / HD * p.log2_base) * 0.15915494309189535f);
    rev -= floorf(rev);
    sn[e] = __builtin_amdgcn_sinf(rev);
    cs[e] = __builtin_amdgcn_cosf(rev);
  }
  float a[8], c[8], sq = 0.f, sk = 0.f;
#pragma unroll
  for (int e = 0; e < 8; e++) a[e] = c[e] = 0.f;
  if (ok) {
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; e++) {
      a[e] = (float)x1[e];
      c[e] = (float)x2[e];
      s += a[e] + c[e];
    }
    sq += which ? 0.f : s;
    sk += which ? s : 0.f;
  }
  float2v sum = wg_sum2_n(sq, sk, red);
  const float mq = sum[0] / D, mk = sum[1] / D;
  sq = sk = 0.f;
  if (ok) {
    const float mean = which ? mk : mq;
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; e++) {
      a[e] -= mean;
      c[e] -= mean;
      s += a[e] * a[e] + c[e] * c[e];
    }
    sq += which ? 0.f : s;
    sk += which ? s : 0.f;
  }
  sum = wg_sum2_n(sq, sk, red);
  const float rq = rsqrtf(sum[0] / D + p.eps), rk = rsqrtf(sum[1] / D + p.eps);
  if (ok) {
    const float rstd = which ? rk : rq;
    const float wl[16] = {w0[0], w0[1], w0[2], w0[3], w1[0], w1[1], w1[2], w1[3],
                          w2[0], w2[1], w2[2], w2[3], w3[0], w3[1], w3[2], w3[3]};
    half8 o1, o2;
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const float x1v = a[e] * rstd * wl[e], x2v = c[e] * rstd * wl[8 + e];
      o1[e] = (half_t)(x1v * cs[e] - x2v * sn[e]);
      o2[e] = (half_t)(x2v * cs[e] + x1v * sn[e]);
    }
    half_t* o = (which ? p.k : p.q) + (((size_t)b * p.H + hh) * p.L + l) * HD + i0;
    st16(o, o1);
    st16(o + HALF, o2);
  }
}

// ---- attention ---------------------------------------------------------------------------------
// One workgroup = 4 waves = 32 queries of one (batch, head). Keys go in passes of LP (256
// or 512; one pass up to L = 512, any length beyond in several, with an online softmax
// carrying each wave's running max, sum and O across passes). Per pass wave w takes keys
// [base + KW w, base + KW (w + 1)) (KW = LP / 4): it streams its K and V rows into a private LDS region
// with buffer loads that write LDS directly, computes S^T = K Q^T for its keys and a
// softmax partial in fp32 (row max m_w, sum l_w, O_w = P V), and the four partials merge
// through LDS: O = sum_w 2^(m_w - M) O_w / sum_w 2^(m_w - M) l_w, M = max_w m_w.
// S^T[key][query] (A = K rows, B = the Q fragments) keeps one query's scores in a lane, so
// the softmax reductions are over registers plus one exchange between the two lane
// halves. Rows 0-7 (and 8-15) of a 32-key block hold keys {4h..4h+3, 8+4h..8+4h+3} (+16):
// a B fragment of O^T = V^T P^T with that k order, so P goes from accumulator to operand
// directly; V^T's A fragments are read from row-major V with ds_read_b64_tr_b16 (4 keys
// of one d per read). LDS key rows are 128 bytes, unpadded (a load writes 64 lanes x 16 B
// to consecutive bytes), with their 16-byte pieces XOR-swizzled: piece p of K row n at
// p ^ ((n >> 1) & 7), so the fragment reads of 16 rows cover the 64 banks once; piece p of
// V row n at p ^ (4 ((n >> 1) & 1)), so the 4 rows x 64 bytes of a transposing read pass do.
// ds_read_b64_tr_b16 of V rows (128 bytes, pieces at p ^ (4 ((n >> 1) & 1))): lane j of a
// 16-lane group names key row k0 + j / 4, d = n0 + 4 (j % 4) .. + 3; lane i receives
// V[k0 + e][n0 + i % 16] for e = 0..3.
DEV half4 tr_read_v(const char* vs, int k0, int n0, int lane) {
  const int j = lane & 15, n = k0 + (j >> 2), d = n0 + 4 * (j & 3);
  return ds_read_tr16x4(vs + n * 128 + 16 * ((d >> 3) ^ (((n >> 1) & 1) << 2)) + 2 * (d & 7));
}

template <int NKB>
__global__ __launch_bounds__(256, NKB <= 8 ? 2 : 1) void esmc_attention_kernel(EsmcAttnArgs p) {
  constexpr int HD = 64, LP = 32 * NKB, KW = LP / 4, KB = KW / 32;  // keys and key blocks per wave
  static_assert(KW % 64 == 0, "whole 64-lane loads of key ids");
  __shared__ __align__(16) char kv_s[4][2 * KW * 128];  // per wave: K rows, then V rows
  __shared__ __align__(16) int sid_s[4][KW];
  __shared__ float ml_s[4][2][32];                       // per wave: m and l of each query

  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 31, h = lane >> 5;
  const int L = p.L;
  // XCD-aware order: the query blocks of one (batch, head) are neighbours, so they run on
  // one XCD and fetch that head's K and V into one L2.
  const int nqb = (p.L + 31) / 32, t = xcd_remap(blockIdx.x, gridDim.x);
  const int bh = t / nqb, b = bh / p.H;
  const int q0 = (t - bh * nqb) * 32;
  const bool has_sid = p.sid != nullptr;
  char* ks = kv_s[wave];
  char* vs = kv_s[wave] + KW * 128;
  const rsrc_t rk = make_rsrc_n(p.k + (size_t)bh * L * HD, (uint32_t)L * HD * 2u);
  const rsrc_t rv = make_rsrc_n(p.v + (size_t)bh * L * HD, (uint32_t)L * HD * 2u);
  const rsrc_t rs = make_rsrc_n(has_sid ? (const void*)(p.sid + (size_t)b * L) : (const void*)p.k,
                                has_sid ? (uint32_t)L * 4u : 0u);

  // Q fragments (B operand: column = query, k = 16 ks + 8 h + e)
  const int qrow = q0 + r;
  half8 qf[HD / 16];
  const rsrc_t rq = make_rsrc_n(p.q + (size_t)bh * L * HD, (uint32_t)L * HD * 2u);
#pragma unroll
  for (int ks4 = 0; ks4 < HD / 16; ks4++) qf[ks4] = bload16(rq, qrow < L ? (uint32_t)(qrow * HD + 16 * ks4 + 8 * h) * 2u : kOOB);
  const int qsid = has_sid && qrow < L ? p.sid[(size_t)b * L + qrow] : 0;

  // The keys go in passes of LP (one pass up to L = LP); per pass wave w takes keys
  // [base + KW w, base + KW (w + 1)), and its running (max, sum, O) are rescaled by
  // 2^(m_old - m_new) when a later pass raises the max (an online softmax).
  float m_run = -INFINITY, sum = 0.f;  // sum: this lane's half of the query's running sum
  f32x16 o[HD / 32];
#pragma unroll
  for (int db = 0; db < HD / 32; db++)
#pragma unroll
    for (int i = 0; i < 16; i++) o[db][i] = 0.f;
  for (int base = 0; base < L; base += LP) {
    const int key0 = base + KW * wave;
    const bool live = key0 < L;  // wave-uniform: a wave past the last key skips the pass
    // the previous pass's LDS reads have all returned before its MFMAs ran; keep the
    // compiler from moving them past the loads that overwrite the rows
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __asm__ volatile("" ::: "memory");
    // K, V rows and key ids of this wave's keys; keys past L load zeros (and are masked).
    if (live) {
#pragma unroll
      for (int i = 0; i < KW / 8; i++) {
        const int n = 8 * i + (lane >> 3), lp = lane & 7;  // row n of this wave's keys, LDS piece lp
        const uint32_t row = (uint32_t)(key0 + n) * 128u;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (__attribute__((address_space(3))) void*)(ks + 1024 * i), 16,
                                                 (int)(row + 16u * (lp ^ ((n >> 1) & 7))), 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (__attribute__((address_space(3))) void*)(vs + 1024 * i), 16,
                                                 (int)(row + 16u * (lp ^ (((n >> 1) & 1) << 2))), 0, 0, 0);
      }
      if (has_sid) {
#pragma unroll
        for (int i = 0; i < KW / 64; i++)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(&sid_s[wave][64 * i]),
                                                   4, (int)((uint32_t)(key0 + 64 * i + lane) * 4u), 0, 0, 0);
      }
    }
    __builtin_amdgcn_s_waitcnt(0x70 | 0xF00);  // vmcnt(0): this wave's LDS rows (and Q) are in
    __asm__ volatile("" ::: "memory");
    if (!live) continue;

    f32x16 sc[KB];
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < KB; kb++) {
#pragma unroll
      for (int i = 0; i < 16; i++) sc[kb][i] = 0.f;
      const int n = 32 * kb + r;
#pragma unroll
      for (int ks4 = 0; ks4 < HD / 16; ks4++) {
        const half8 kf = *reinterpret_cast<const half8*>(ks + n * 128 + 16 * ((2 * ks4 + h) ^ ((n >> 1) & 7)));
        sc[kb] = mfma32(kf, qf[ks4], sc[kb]);
      }
#pragma unroll
      for (int i4 = 0; i4 < 4; i4++) {
        const int kl = 32 * kb + acc_row32(4 * i4, lane);  // 4 consecutive keys of this wave
        int4 sid4 = {0, 0, 0, 0};
        if (has_sid) sid4 = *reinterpret_cast<const int4*>(&sid_s[wave][kl]);
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int i = 4 * i4 + e;
          const bool ok = key0 + kl + e < L && sid4[e] == qsid;
          sc[kb][i] = ok ? sc[kb][i] * p.scale_log2 : -INFINITY;
          mx = fmaxf(mx, sc[kb][i]);
        }
      }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const float mref = m_new == -INFINITY ? 0.f : m_new;  // no key visible to the query yet
    const float alpha = __builtin_amdgcn_exp2f(m_run - mref);  // 0 on the first visible pass
    sum *= alpha;
#pragma unroll
    for (int db = 0; db < HD / 32; db++)
#pragma unroll
      for (int i = 0; i < 16; i++) o[db][i] *= alpha;
    m_run = m_new;
    half8 pf[2 * KB];
#pragma unroll
    for (int kb = 0; kb < KB; kb++)
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const float e = __builtin_amdgcn_exp2f(sc[kb][i] - mref);  // (v_exp_f32: results below 2^-126 flush)
        sum += e;
        pf[2 * kb + (i >> 3)][i & 7] = (half_t)e;
      }
    // O^T[d][query] += sum over this wave's keys of V^T[d][key] P[key][query]
    const int n0q = 16 * ((lane >> 4) & 1);  // d offset of this lane's 16-lane group
#pragma unroll
    for (int j = 0; j < 2 * KB; j++) {
#pragma unroll
      for (int db = 0; db < HD / 32; db++) {
        const half4 lo = tr_read_v(vs, 16 * j + 4 * h, 32 * db + n0q, lane);
        const half4 hi = tr_read_v(vs, 16 * j + 8 + 4 * h, 32 * db + n0q, lane);
        o[db] = mfma32(half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]}, pf[j], o[db]);
      }
    }
  }
  const float mx = m_run;
  sum += __shfl_xor(sum, 32);

  // Partials -> LDS: m, l per query; O_w in accumulator order over this wave's K rows
  // (8 quads x 64 lanes x 16 B = 8 KB, no longer read by anyone).
  if (h == 0) {
    ml_s[wave][0][r] = mx;
    ml_s[wave][1][r] = sum;
  }
  f32x4* ow = reinterpret_cast<f32x4*>(ks);
#pragma unroll
  for (int db = 0; db < HD / 32; db++)
#pragma unroll
    for (int r4 = 0; r4 < 4; r4++)
      ow[(4 * db + r4) * 64 + lane] = f32x4{o[db][4 * r4], o[db][4 * r4 + 1], o[db][4 * r4 + 2], o[db][4 * r4 + 3]};
  __syncthreads();

  // Wave w finishes quads 2w, 2w + 1: d = 32 db + acc_row32(4 r4, lane) .. + 3 of query r.
  if (qrow < L) {
    float m4[4], M = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; w++) {
      m4[w] = ml_s[w][0][r];
      M = fmaxf(M, m4[w]);
    }
    float den = 0.f, sc[4];
#pragma unroll
    for (int w = 0; w < 4; w++) {
      sc[w] = __builtin_amdgcn_exp2f(m4[w] - M);  // 0 for a wave that saw no visible key
      den += sc[w] * ml_s[w][1][r];
    }
    const float inv = 1.0f / den;
    half_t* dst = p.o + ((size_t)b * L + qrow) * (p.H * HD) + (bh - b * p.H) * HD;
#pragma unroll
    for (int u = 0; u < 2; u++) {
      const int qd = 2 * wave + u, db = qd >> 2, r4 = qd & 3;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int w = 0; w < 4; w++) acc += sc[w] * reinterpret_cast<const f32x4*>(kv_s[w])[qd * 64 + lane];
      const int d = 32 * db + acc_row32(4 * r4, lane);
      *reinterpret_cast<half4*>(dst + d) =
          half4{(half_t)(acc[0] * inv), (half_t)(acc[1] * inv), (half_t)(acc[2] * inv), (half_t)(acc[3] * inv)};
    }
  }
}

// ---- SwiGLU --------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void esmc_swiglu_kernel(const half_t* __restrict__ x12, half_t* __restrict__ y,
                                                          size_t M, int F) {
  const size_t n8 = M * (size_t)(F / 8);
  for (size_t c = (size_t)blockIdx.x * blockDim.x + threadIdx.x; c < n8; c += (size_t)gridDim.x * blockDim.x) {
    const size_t m = c / (F / 8);
    const int f0 = 8 * (int)(c - m * (F / 8));
    const half8 a = ld16(x12 + m * 2 * F + f0), g = ld16(x12 + m * 2 * F + F + f0);
    half8 o;
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const float u = (float)a[e];
      o[e] = (half_t)(u * sigmoidf_fast(u) * (float)g[e]);
    }
    st16(y + m * F + f0, o);
  }
}

template <int NJ>
static hipError_t launch_esmc_ln_nj(const EsmcLnArgs& a, hipStream_t s) {
  const int ns = a.yp ? a.splits : 0;
  if (ns == 4)
    ESM_LAUNCH((esmc_ln_kernel<NJ, 4>), dim3(a.M), dim3(NTR), 0, s, a);
  else if (ns == 3)
    ESM_LAUNCH((esmc_ln_kernel<NJ, 3>), dim3(a.M), dim3(NTR), 0, s, a);
  else if (ns == 2)
    ESM_LAUNCH((esmc_ln_kernel<NJ, 2>), dim3(a.M), dim3(NTR), 0, s, a);
  else if (ns == 1)
    ESM_LAUNCH((esmc_ln_kernel<NJ, 1>), dim3(a.M), dim3(NTR), 0, s, a);
  else  // no partials (NSPL is then unused), or another count
    ESM_LAUNCH((esmc_ln_kernel<NJ, -1>), dim3(a.M), dim3(NTR), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_esmc_ln(const EsmcLnArgs& a, hipStream_t s) {
  switch ((a.D + 4 * NTR - 1) / (4 * NTR)) {  // element groups per thread
    case 1: return launch_esmc_ln_nj<1>(a, s);
    case 2: return launch_esmc_ln_nj<2>(a, s);
    case 3: return launch_esmc_ln_nj<3>(a, s);
    case 4: return launch_esmc_ln_nj<4>(a, s);
    case 5: return launch_esmc_ln_nj<5>(a, s);
    case 6: return launch_esmc_ln_nj<6>(a, s);
    case 7: return launch_esmc_ln_nj<7>(a, s);
    case 8: return launch_esmc_ln_nj<8>(a, s);
    default: return hipErrorInvalidValue;  // D <= 8192 is checked by the caller
  }
}

hipError_t launch_esmc_qk_rope(const EsmcRopeArgs& a, hipStream_t s) {
  const int D = a.H * 64, chunks = 2 * (D / 16) > D / 8 ? 2 * (D / 16) : D / 8;  // q/k chunks, v chunks
  const int nthr = (chunks + 63) / 64 * 64;
  if (nthr > kRopeMaxThreads) return hipErrorInvalidValue;  // D <= 4096 is checked by the caller
  ESM_LAUNCH(esmc_qk_rope_kernel, dim3(a.B * a.L), dim3(nthr), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_esmc_attention(const EsmcAttnArgs& a, hipStream_t s) {
  const dim3 grid(((a.L + 31) / 32) * a.B * a.H);
  if (a.L <= 256)  // one pass of 256 keys; longer sequences take passes of 512
    ESM_LAUNCH(esmc_attention_kernel<8>, grid, dim3(256), 0, s, a);
  else
    ESM_LAUNCH(esmc_attention_kernel<16>, grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_esmc_swiglu(const half_t* x12, half_t* y, size_t M, int F, hipStream_t s) {
  const size_t n8 = M * (size_t)(F / 8), blocks = (n8 + 255) / 256;
  ESM_LAUNCH(esmc_swiglu_kernel, dim3((unsigned)(blocks < 4096 ? blocks : 4096)), dim3(256), 0, s, x12, y, M, F);
  return hipGetLastError();
}

}  // namespace esm
