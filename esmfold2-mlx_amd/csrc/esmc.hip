// Kernels of the ESMC transformer block around the 8-bit linear (mlx_esmc.py:84-102),
// other than the q8 GEMMs themselves (q8.hip):
//   esmc_ln        x' = x + alpha*y (fp32 residual, optional), h = LN(x') -> fp16 or fp32
//   esmc_qk_rope   QK-LayerNorm over the full width (weight only, fp32 statistics),
//                  NeoX rotary embedding, head-major q, k, v for the attention
//   esmc_attention softmax(q k^T * scale, same-chain mask) v, one head per workgroup
//                  column, MFMA for both products
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

// ---- residual + LayerNorm -------------------------------------------------------------------
__global__ __launch_bounds__(NTR) void esmc_ln_kernel(EsmcLnArgs p) {
  __shared__ float red[4];
  const int row = blockIdx.x, D = p.D;
  const float* x = p.x + (size_t)row * D;
  float* xo = p.x_out + (size_t)row * D;
  const half_t* y = p.y ? p.y + (size_t)row * D : nullptr;
  half_t* h = p.h ? p.h + (size_t)row * D : nullptr;
  float* h32 = p.h32 ? p.h32 + (size_t)row * D : nullptr;
  constexpr int MAXV = 8;  // D <= 8 * 4 * 256
  f32x4 v[MAXV];
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < MAXV; j++) {
    const int i = 4 * (threadIdx.x + NTR * j);
    if (i < D) {
      f32x4 t = *reinterpret_cast<const f32x4*>(x + i);
      if (y) {
        const half4 yy = *reinterpret_cast<const half4*>(y + i);
#pragma unroll
        for (int e = 0; e < 4; e++) t[e] += p.alpha * (float)yy[e];
        *reinterpret_cast<f32x4*>(xo + i) = t;
      }
      v[j] = t;
      s += t[0] + t[1] + t[2] + t[3];
    }
  }
  const float mean = wg_sum(s, red) / D;
  float q = 0.f;
#pragma unroll
  for (int j = 0; j < MAXV; j++) {
    const int i = 4 * (threadIdx.x + NTR * j);
    if (i < D)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        v[j][e] -= mean;
        q += v[j][e] * v[j][e];
      }
  }
  const float rstd = rsqrtf(wg_sum(q, red) / D + p.eps);
#pragma unroll
  for (int j = 0; j < MAXV; j++) {
    const int i = 4 * (threadIdx.x + NTR * j);
    if (i < D) {
      f32x4 o;
#pragma unroll
      for (int e = 0; e < 4; e++) o[e] = v[j][e] * rstd * p.w[i + e] + (p.b ? p.b[i + e] : 0.f);
      if (h) *reinterpret_cast<half4*>(h + i) = half4{(half_t)o[0], (half_t)o[1], (half_t)o[2], (half_t)o[3]};
      if (h32) *reinterpret_cast<f32x4*>(h32 + i) = o;
    }
  }
}

// ---- QK-LayerNorm + RoPE, head-major outputs ---------------------------------------------------
// Thread -> rotation pairs (e, e + hd/2) of one head: pair index u = tid + 256 j,
// head = u / (hd/2), i = u % (hd/2). hd = 64.
__global__ __launch_bounds__(NTR) void esmc_qk_rope_kernel(EsmcRopeArgs p) {
  __shared__ float red[4];
  constexpr int HD = 64, HALF = 32, MAXP = 8;  // D <= 8 * 256 * 2
  const int row = blockIdx.x, D = p.H * HD;
  const int b = row / p.L, l = row - b * p.L;
  const half_t* src = p.qkv + (size_t)row * 3 * D;
  const int npairs = D / 2;
  // rotation angles of this thread's pairs: l * base^(-2i/hd)
  float cs[MAXP], sn[MAXP];
#pragma unroll
  for (int j = 0; j < MAXP; j++) {
    const int u = threadIdx.x + NTR * j;
    const int i = u % HALF;
    const float ang = (float)l * exp2f(-(float)(2 * i) / HD * p.log2_base);
    sincosf(ang, &sn[j], &cs[j]);
  }
#pragma unroll
  for (int which = 0; which < 2; which++) {  // 0: q, 1: k
    const half_t* v = src + which * D;
    const float* w = which ? p.k_ln : p.q_ln;
    half_t* dst = which ? p.k : p.q;
    float a[MAXP], c[MAXP], s = 0.f;
#pragma unroll
    for (int j = 0; j < MAXP; j++) {
      const int u = threadIdx.x + NTR * j;
      a[j] = c[j] = 0.f;
      if (u < npairs) {
        const int e = (u / HALF) * HD + (u % HALF);
        a[j] = (float)v[e];
        c[j] = (float)v[e + HALF];
        s += a[j] + c[j];
      }
    }
    const float mean = wg_sum(s, red) / D;
    float q = 0.f;
#pragma unroll
    for (int j = 0; j < MAXP; j++) {
      const int u = threadIdx.x + NTR * j;
      if (u < npairs) {
        a[j] -= mean;
        c[j] -= mean;
        q += a[j] * a[j] + c[j] * c[j];
      }
    }
    const float rstd = rsqrtf(wg_sum(q, red) / D + p.eps);
#pragma unroll
    for (int j = 0; j < MAXP; j++) {
      const int u = threadIdx.x + NTR * j;
      if (u < npairs) {
        const int hh = u / HALF, i = u % HALF, e = hh * HD + i;
        const float x1 = a[j] * rstd * w[e], x2 = c[j] * rstd * w[e + HALF];
        half_t* o = dst + (((size_t)b * p.H + hh) * p.L + l) * HD;
        o[i] = (half_t)(x1 * cs[j] - x2 * sn[j]);
        o[i + HALF] = (half_t)(x2 * cs[j] + x1 * sn[j]);
      }
    }
  }
  // v: copy to head-major, 8 halfs per thread
  for (int c8 = threadIdx.x; c8 < D / 8; c8 += NTR) {
    const int e = 8 * c8, hh = e / HD, d = e % HD;
    st16(p.v + (((size_t)b * p.H + hh) * p.L + l) * HD + d, ld16(src + 2 * D + e));
  }
}

// ---- attention ---------------------------------------------------------------------------------
// One workgroup = 4 waves = 128 queries of one (batch, head); each wave 32 queries.
// S^T[key][query] = K Q^T (A = K rows from LDS, B = the wave's Q fragments), so a lane
// holds one query's scores: the softmax reductions are over registers plus one exchange
// between the two lane halves. Rows 0-7 (and 8-15) of a 32-key block hold keys
// {4h..4h+3, 8+4h..8+4h+3} (+16): a B fragment of O^T = V^T P^T with that k order, so P
// goes from accumulator to operand directly; V^T's fragments are read in the same order.
template <int NKB>
__global__ __launch_bounds__(256, 1) void esmc_attention_kernel(EsmcAttnArgs p) {
  constexpr int HD = 64, LP = 32 * NKB;           // keys padded to whole blocks
  constexpr int KSTR = HD + 8;                     // K rows in LDS (halfs): 144 B, conflict-free
  constexpr int VSTR = LP + 8;                     // V^T rows in LDS (halfs)
  __shared__ __align__(16) half_t k_s[LP * KSTR];
  __shared__ __align__(16) half_t vt_s[HD * VSTR];
  __shared__ int sid_s[LP];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 31, h = lane >> 5;
  const int L = p.L;
  const int bh = blockIdx.y, b = bh / p.H;
  const int q0 = blockIdx.x * 128 + wave * 32;
  const half_t* Q = p.q + (size_t)bh * L * HD;
  const half_t* K = p.k + (size_t)bh * L * HD;
  const half_t* V = p.v + (size_t)bh * L * HD;

  // K -> LDS rows, V -> LDS transposed; keys past L are zero. Every load is issued before
  // the first LDS write (a rolled loop waited on each iteration's loads in turn).
  constexpr int NCH = LP * (HD / 8) / 256;  // 16-byte chunks of K (and of V) per thread
  static_assert(LP * (HD / 8) % 256 == 0, "whole chunks per thread");
  const rsrc_t rk = make_rsrc(K), rv = make_rsrc(V);
  half8 kv[NCH], vv[NCH];
#pragma unroll
  for (int i = 0; i < NCH; i++) {
    const int c = tid + 256 * i, key = c / (HD / 8), d0 = 8 * (c % (HD / 8));
    const uint32_t off = key < L ? (uint32_t)(key * HD + d0) * 2u : kOOB;
    kv[i] = bload16(rk, off);
    vv[i] = bload16(rv, off);
  }
#pragma unroll
  for (int i = 0; i < NCH; i++) {
    const int c = tid + 256 * i, key = c / (HD / 8), d0 = 8 * (c % (HD / 8));
    st16(&k_s[key * KSTR + d0], kv[i]);
#pragma unroll
    for (int e = 0; e < 8; e++) vt_s[(d0 + e) * VSTR + key] = vv[i][e];
  }
  for (int key = tid; key < LP; key += 256) sid_s[key] = key < L ? (p.sid ? p.sid[(size_t)b * L + key] : 0) : -2;
  __syncthreads();
  if (q0 >= L) return;  // a wave past the last query (no later barrier)

  // this wave's Q fragments (B operand: column = query, k = 16 ks + 8 h + e)
  const int qrow = q0 + r;
  half8 qf[HD / 16];
#pragma unroll
  for (int ks = 0; ks < HD / 16; ks++) qf[ks] = qrow < L ? ld16(Q + (size_t)qrow * HD + 16 * ks + 8 * h) : zero_half8();
  const int qsid = qrow < L ? (p.sid ? p.sid[(size_t)b * L + qrow] : 0) : -3;

  const int nkb = (L + 31) / 32;
  f32x16 s[NKB];
  float mx = -INFINITY;
#pragma unroll
  for (int kb = 0; kb < NKB; kb++) {
    if (kb < nkb) {
#pragma unroll
      for (int i = 0; i < 16; i++) s[kb][i] = 0.f;
#pragma unroll
      for (int ks = 0; ks < HD / 16; ks++)
        s[kb] = mfma32(ld16(&k_s[(32 * kb + r) * KSTR + 16 * ks + 8 * h]), qf[ks], s[kb]);
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const int key = 32 * kb + acc_row32(i, lane);
        const bool ok = key < L && sid_s[key] == qsid;
        s[kb][i] = ok ? s[kb][i] * p.scale_log2 : -INFINITY;
        mx = fmaxf(mx, s[kb][i]);
      }
    }
  }
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  float sum = 0.f;
  half8 pf[2 * NKB];
#pragma unroll
  for (int kb = 0; kb < NKB; kb++) {
    if (kb < nkb) {
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const float e = exp2f(s[kb][i] - mx);
        sum += e;
        pf[2 * kb + (i >> 3)][i & 7] = (half_t)e;
      }
    }
  }
  sum += __shfl_xor(sum, 32);

  // O^T[d][query] = sum over keys of V^T[d][key] P[key][query]
  f32x16 o[HD / 32];
#pragma unroll
  for (int db = 0; db < HD / 32; db++)
#pragma unroll
    for (int i = 0; i < 16; i++) o[db][i] = 0.f;
#pragma unroll
  for (int j = 0; j < 2 * NKB; j++) {
    if (j < 2 * nkb) {
      const int k0 = 16 * j + 4 * h;
#pragma unroll
      for (int db = 0; db < HD / 32; db++) {
        const half_t* vr = &vt_s[(32 * db + r) * VSTR];
        const half4 lo = *reinterpret_cast<const half4*>(vr + k0);
        const half4 hi = *reinterpret_cast<const half4*>(vr + k0 + 8);
        o[db] = mfma32(half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]}, pf[j], o[db]);
      }
    }
  }
  if (qrow < L) {
    const float inv = 1.0f / sum;
    half_t* dst = p.o + ((size_t)b * L + qrow) * (p.H * HD) + (bh - b * p.H) * HD;
#pragma unroll
    for (int db = 0; db < HD / 32; db++)
#pragma unroll
      for (int r4 = 0; r4 < 4; r4++) {
        const int d = 32 * db + acc_row32(4 * r4, lane);
        *reinterpret_cast<half4*>(dst + d) = half4{(half_t)(o[db][4 * r4] * inv), (half_t)(o[db][4 * r4 + 1] * inv),
                                                   (half_t)(o[db][4 * r4 + 2] * inv), (half_t)(o[db][4 * r4 + 3] * inv)};
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

hipError_t launch_esmc_ln(const EsmcLnArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(esmc_ln_kernel, dim3(a.M), dim3(NTR), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_esmc_qk_rope(const EsmcRopeArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(esmc_qk_rope_kernel, dim3(a.B * a.L), dim3(NTR), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_esmc_attention(const EsmcAttnArgs& a, hipStream_t s) {
  const dim3 grid((a.L + 127) / 128, a.B * a.H);
  if (a.L <= 256)
    hipLaunchKernelGGL(esmc_attention_kernel<8>, grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(esmc_attention_kernel<16>, grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_esmc_swiglu(const half_t* x12, half_t* y, size_t M, int F, hipStream_t s) {
  const size_t n8 = M * (size_t)(F / 8), blocks = (n8 + 255) / 256;
  hipLaunchKernelGGL(esmc_swiglu_kernel, dim3((unsigned)(blocks < 4096 ? blocks : 4096)), dim3(256), 0, s, x12, y, M, F);
  return hipGetLastError();
}

}  // namespace esm
