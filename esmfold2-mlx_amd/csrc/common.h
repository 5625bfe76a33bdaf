// Shared device helpers for the gfx950 (CDNA4) kernels: vector types, MFMA
// wrappers, LayerNorm statistics and reductions, buffer access and weight staging.
//
// MFMA lane layouts used throughout (checked on an MI355X by an in-bounds
// probe before any kernel relied on them):
//   v_mfma_f32_32x32x16_f16(a, b, c):
//     a: 8 halfs per lane, row  = lane % 32, k = 8*(lane/32) + e   (A is 32x16)
//     b: 8 halfs per lane, col  = lane % 32, k = 8*(lane/32) + e   (B is 16x32)
//     c/d: 16 floats per lane, col = lane % 32,
//          row = 8*(r/4) + 4*(lane/32) + (r%4) for register r.
//   A GEMM only needs A and B to agree on the k assignment, so "k = 8*(lane/32)+e"
//   is a convention both operands follow.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

// --- launch timing (host side) ----------------------------------------------------------
// While esm_timing_begin has armed the calling thread, each launch made through ESM_LAUNCH
// takes the next pair of pre-created events and hands them to hipExtLaunchKernelGGL, which
// stamps the kernel's own start and end into them: the elapsed times are the kernels'
// durations as a profiler's kernel trace reports them, without the dispatch time an event
// pair recorded around a launch adds. Unarmed, ESM_LAUNCH is hipLaunchKernelGGL.
namespace esm {
bool timing_slot(const char* kernel_name, hipEvent_t* start, hipEvent_t* stop);
}
#define ESM_LAUNCH(kernel, grid, block, lds, stream, ...)                                          \
  do {                                                                                             \
    hipEvent_t esm_t0_, esm_t1_;                                                                   \
    if (esm::timing_slot(#kernel, &esm_t0_, &esm_t1_))                                             \
      hipExtLaunchKernelGGL(kernel, grid, block, lds, stream, esm_t0_, esm_t1_, 0, __VA_ARGS__);   \
    else                                                                                           \
      hipLaunchKernelGGL(kernel, grid, block, lds, stream, __VA_ARGS__);                           \
  } while (0)

typedef _Float16 half_t;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#define DEV __device__ __forceinline__

DEV f32x16 mfma32(half8 a, half8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

DEV f32x4 mfma16(half8 a, half8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Row of the 32x32 MFMA accumulator held by register r of this lane.
DEV int acc_row32(int r, int lane) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }

DEV half8 ld16(const half_t* p) { return *reinterpret_cast<const half8*>(p); }

// --- buffer (descriptor-based) global access -----------------------------------------
// A raw buffer resource with a wave-uniform base and a 2 GB range. A lane whose byte
// offset is kOOB (>= the range) is out of bounds: its load returns zeros and its store is
// dropped by the hardware. Guarding with kOOB instead of a branch keeps every memory
// instruction unconditional, so the compiler can count outstanding loads exactly and a
// prefetch issued one tile ahead really stays in flight.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr uint32_t kOOB = 0x80000000u;
constexpr int kBufRange = 0x7ffffff0;
// Word 3 of a gfx9-family (CDNA) raw buffer descriptor: 32-bit data format, no swizzle.
constexpr int kBufWord3 = 0x00020000;

DEV rsrc_t make_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, kBufRange, kBufWord3);
}
// A raw buffer resource whose range is exactly `bytes`: any offset at or past it
// (including kOOB) loads zeros.
DEV rsrc_t make_rsrc_n(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kBufWord3);
}
DEV half8 bload16(rsrc_t r, uint32_t off) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
  return __builtin_bit_cast(half8, v);
}
DEV void bstore16(rsrc_t r, uint32_t off, half8 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, (int)off, 0, 0);
}
DEV void bstore8(rsrc_t r, uint32_t off, half4 v) {
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, v), r, (int)off, 0, 0);
}
DEV uint16_t bload2(rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, 0); }
DEV float h2f(uint16_t bits) { return (float)__builtin_bit_cast(half_t, bits); }
DEV void st16(half_t* p, half8 v) { *reinterpret_cast<half8*>(p) = v; }

DEV half8 zero_half8() {
  half8 v;
#pragma unroll
  for (int e = 0; e < 8; e++) v[e] = (half_t)0.0f;
  return v;
}

// Sum over the 16 lanes of a DPP row (lanes 16k .. 16k+15); every lane gets the sum.
// DPP row rotations (row_ror:8, 4, 2, 1) stay in the VALU: no LDS round trip per step.
// After rotating by 8, 4, 2 and 1 and adding, each lane has added all 16 lanes once.
template <int CTRL>
DEV float dpp_f32(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
DEV float row16_sum(float v) {
  v += dpp_f32<0x128>(v);  // row_ror:8
  v += dpp_f32<0x124>(v);  // row_ror:4
  v += dpp_f32<0x122>(v);  // row_ror:2
  v += dpp_f32<0x121>(v);  // row_ror:1
  return v;
}

// --- workgroup order --------------------------------------------------------------------
// The dispatcher deals workgroup ids round-robin to the 8 XCDs (each with its own L2).
// This bijection of [0, n) gives each XCD a contiguous run of logical indices, so
// logical neighbours that read the same operands share one L2.
constexpr int kNumXcd = 8;
DEV int xcd_remap(int id, int n) {
  const int per = n / kNumXcd, rem = n % kNumXcd;
  const int xcd = id % kNumXcd, slot = id / kNumXcd;
  return xcd < rem ? xcd * (per + 1) + slot : rem * (per + 1) + (xcd - rem) * per + slot;
}

// --- weight staging ----------------------------------------------------------------------
// Weight rows of 128 halfs (256 B) go through LDS so that the global reads are fully
// coalesced (each load instruction of a workgroup covers NT*16 contiguous bytes). Read
// straight into MFMA fragments, every instruction would touch 32 different rows, and the
// per-CU L1 path would need several times as many cycles for the same bytes. In LDS the
// 16-byte chunk j of row r sits at chunk j ^ (r & 15): the fragment reads of 16
// consecutive rows at one logical chunk hit 16 distinct chunk positions (all 64 banks).
template <int ROWS, int NT>
struct RowStage {
  static constexpr int kPer = ROWS * 16 / NT;  // 16-byte chunks per thread
  static_assert(ROWS * 16 % NT == 0, "whole chunks per thread");
  half8 v[kPer];
  DEV void load(const half_t* src, int tid) {
#pragma unroll
    for (int i = 0; i < kPer; i++) v[i] = ld16(src + 8 * (tid + NT * i));
  }
  DEV void store(half_t* dst, int tid) const {
#pragma unroll
    for (int i = 0; i < kPer; i++) {
      const int q = tid + NT * i, r = q >> 4, j = q & 15;
      st16(dst + r * 128 + 8 * (j ^ (r & 15)), v[i]);
    }
  }
};
// Logical 16-byte chunk j (halfs 8j .. 8j+7) of staged row r.
DEV half8 staged_chunk(const half_t* s, int r, int j) { return ld16(s + r * 128 + 8 * (j ^ (r & 15))); }

// -log2(e): with t = -x log2(e), sigmoid(x) = 1 / (1 + 2^t).
constexpr float kNegLog2e = -1.4426950408889634f;
// sigmoid from t = -x log2(e): v_exp_f32, one add, v_rcp_f32.
DEV float sigmoid_from_t(float t) { return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(t)); }

DEV float sigmoidf_fast(float x) {
  // 1 / (1 + e^-x): v_exp_f32 and v_rcp_f32 (about 1 ulp each); saturates
  // cleanly to 0 and 1 at +-inf.
  return __builtin_amdgcn_rcpf(1.0f + __expf(-x));
}

// --- LayerNorm from fp16 inputs, three VALU operations per value ----------------------
// Sums of the values and of their squares, accumulated in fp32: v_dot2_f32_f16 forms two
// exact fp16 products per instruction (the sum: products with 1).
DEV void dot2_moments(half8 v, float& s, float& q) {
  const half2v one = {(half_t)1.0f, (half_t)1.0f};
#pragma unroll
  for (int p = 0; p < 4; p++) {
    const half2v x = {v[2 * p], v[2 * p + 1]};
    s = __builtin_amdgcn_fdot2(x, one, s, false);
    q = __builtin_amdgcn_fdot2(x, x, q, false);
  }
}
DEV void dot2_moments(half4 v, float& s, float& q) {
  const half2v one = {(half_t)1.0f, (half_t)1.0f};
#pragma unroll
  for (int p = 0; p < 2; p++) {
    const half2v x = {v[2 * p], v[2 * p + 1]};
    s = __builtin_amdgcn_fdot2(x, one, s, false);
    q = __builtin_amdgcn_fdot2(x, x, q, false);
  }
}
// gfx950's transposing LDS read, ds_read_b64_tr_b16: in each 16-lane group, lane j names the
// 8-byte piece P_j (4 fp16 values) at p, and lane n receives P_{4e + n/4}[n % 4], e = 0..3.
// With P_j = row r0 + j/4, columns c0 + 4 (j % 4) .. +3 of a row-major tile, lane n gets
// column c0 + n of rows r0 .. r0+3.
typedef short v4s_t __attribute__((ext_vector_type(4)));
DEV half4 ds_read_tr16x4(const void* p) {
  const v4s_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) v4s_t*)(__attribute__((address_space(3))) const char*)p);
  return __builtin_bit_cast(half4, v);
}

// rstd = 1 / sqrt(var + eps) and shift = -mean * rstd from the sums over n values, with
// var = E[x^2] - E[x]^2 in fp32 (clamped at 0). Against the two-pass form this loses about
// n 2^-24 (1 + mean^2 / var) of var: below the fp16 rounding of the result while |mean| is
// within 8 standard deviations of a row.
DEV void ln_scale_shift(float s, float q, float inv_n, float eps, float& rstd, float& shift) {
  const float mean = s * inv_n;
  const float var = fmaxf(fmaf(q, inv_n, -mean * mean), 0.f);
  rstd = rsqrtf(var + eps);
  shift = -mean * rstd;
}
// One normalised value, (x - mean) rstd gamma + beta, from its fp16 input (v_fma_mix_f32
// reads the fp16 operand directly), rounded once to fp16. The fp32 result is materialised
// first: otherwise the compiler may fold the conversion into the last FMA in one inlined
// copy and not in another, and the same value would round differently by position.
DEV half_t ln_value(half_t x, float rstd, float shift, float g, float b) {
  float y = fmaf(fmaf((float)x, rstd, shift), g, b);
  __asm__ volatile("" : "+v"(y));
  return (half_t)y;
}

// LayerNorm of one 8-channel slice held by this lane, where the 16 lanes of a DPP row
// together hold one 128-channel row: fp16 in, fp16 out, fp32 statistics (dot2_moments).
DEV half8 ln_row128_h(half8 x, const float (&g)[8], const float (&b)[8], float eps) {
  float s = 0.f, q = 0.f;
  dot2_moments(x, s, q);
  s = row16_sum(s);
  q = row16_sum(q);
  float rstd, shift;
  ln_scale_shift(s, q, 1.0f / 128.0f, eps, rstd, shift);
  half8 o;
#pragma unroll
  for (int e = 0; e < 8; e++) o[e] = ln_value(x[e], rstd, shift, g[e], b[e]);
  return o;
}
