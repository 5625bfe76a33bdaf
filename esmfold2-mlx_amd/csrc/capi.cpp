// C ABI (include/esmfold2_amd.h): argument validation, launch geometry and
// error reporting around the gfx950 kernels. Nothing here allocates device
// memory; every launch goes on the caller's stream.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/esmfold2_amd.h"
#include "kernels.h"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int ok() {
  g_err.clear();
  return ESM_OK;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return ok();
  return fail((int)e, "%s: %s", what, hipGetErrorString(e));
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Compute units of the current device (persistent-grid sizing), cached per device.
int cu_count() {
  static std::mutex mu;
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::lock_guard<std::mutex> lk(mu);
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// Pair side limit. Every kernel addresses its tile, line or channel plane from a 64-bit base,
// so nothing bounds B * L * L * C but memory; what L bounds is the 32-bit offset within one
// such base: kernel (a) writes 32 channel planes of a fragment-layout tile from one base
// (32 x 2 x L^2 bytes: 1.07 GB at 4096) and kernel (c) reads 16 channel rows (0.5 GB).
constexpr int kMaxL = 4096;

// q8 GEMM launch plan. A tile is kQ8TileM x 32 nb outputs, nb = 4 (128 weight rows) or 5
// (160). When the tiles alone cannot fill the GPU, K is split over up to kQ8MaxSplits
// workgroups per tile (each of the 4 waves keeps at least one 64-wide group) and the
// partials go through the caller's workspace: [splits, M, N] fp32, summed by a second
// kernel. The width is the one with the lower estimate of rounds x steps per workgroup x
// the time of a step (a 128-row step takes ~0.9 of a 160-row one, ~0.7 us at K = 2560 on
// 256 CUs), plus, when K is split, writing and reading back the partials (~4 TB/s).
// Measured at M = 238, 128 against 160 rows: N = 7680 unsplit 20.8 against 22.5 us (also
// inside the ESMC block's graph); N = 2560 split at K = 2560 10.9 against 11.2 in the graph
// (16.6 against 19.1 alone with the reduction kernel), at K = 5120 16.0 against 15.3 in the
// graph (21.2 against 22.2 alone), at K = 10240 31.8 against 29.4 alone; N = 10240 takes 160
// rows (256 tiles, one round; 320 at 128 rows). A SwiGLU-pair weight always takes the wide tile, whose 80 + 80
// rows the pair order is laid out for.
constexpr int kQ8MaxSplits = 16;
constexpr int kQ8MaxK = 1 << 20;  // keeps every per-row byte offset far below 2^31
constexpr double kQ8StepUs = 0.7, kQ8NarrowStep = 0.9, kQ8PartialBytesPerUs = 4.0e6;
std::atomic<int> g_q8_tile_rows{0};  // q8_set_tile_rows: 0 lets the plan choose
struct Q8Plan {
  int mtiles, ntiles, splits, nb;
  size_t bytes;
};
Q8Plan q8_plan_nb(int M, int K, int N, int nb) {
  Q8Plan p;
  p.nb = nb;
  p.mtiles = (M + esm::kQ8TileM - 1) / esm::kQ8TileM;
  p.ntiles = (N + 32 * nb - 1) / (32 * nb);
  const long long tiles = (long long)p.mtiles * p.ntiles;
  const int groups = K / 64;
  long long sp = cu_count() / tiles;
  if (sp > kQ8MaxSplits) sp = kQ8MaxSplits;
  if (sp > groups / esm::kQ8Waves) sp = groups / esm::kQ8Waves;
  p.splits = sp < 1 ? 1 : (int)sp;
  p.bytes = (size_t)p.splits * M * N * sizeof(float);
  return p;
}
double q8_plan_cost(const Q8Plan& p, int M, int K, int N) {
  const long long cus = cu_count(), wgs = (long long)p.mtiles * p.ntiles * p.splits;
  const long long rounds = (wgs + cus - 1) / cus, steps = ((K / 64 + 1) / 2 + p.splits - 1) / p.splits;
  double c = (double)rounds * (double)steps * kQ8StepUs * (p.nb == esm::kQ8TileNbWide ? 1.0 : kQ8NarrowStep);
  if (p.splits > 1) c += p.splits * (double)M * N * 8.0 / kQ8PartialBytesPerUs;
  return c;
}
Q8Plan q8_plan(int M, int K, int N, bool swiglu = false) {
  const int forced = g_q8_tile_rows.load() / 32;
  if (swiglu) return q8_plan_nb(M, K, N, esm::kQ8TileNbWide);
  if (forced) return q8_plan_nb(M, K, N, forced);
  const Q8Plan narrow = q8_plan_nb(M, K, N, esm::kQ8TileNbNarrow), wide = q8_plan_nb(M, K, N, esm::kQ8TileNbWide);
  return q8_plan_cost(narrow, M, K, N) <= q8_plan_cost(wide, M, K, N) ? narrow : wide;
}

#ifndef ESM_SOURCE_HASH
#define ESM_SOURCE_HASH "unknown"
#endif
// The content hash of the sources this library was built from, also findable as a tagged
// string in the file itself, so a loader can tell a stale build without loading it.
__attribute__((used)) const char kSourceTag[] = "ESMSRC:" ESM_SOURCE_HASH;

using esm::half_t;
inline const half_t* H(const esm_half* p) { return reinterpret_cast<const half_t*>(p); }
inline half_t* H(esm_half* p) { return reinterpret_cast<half_t*>(p); }

int round_up(int v, int m) { return (v + m - 1) / m * m; }

}  // namespace

// Launch timing state (see ESM_LAUNCH in common.h): events created once and reused; a
// session hands them out pairwise, in launch order, until esm_timing_end.
namespace {
struct TimingSession {
  std::vector<hipEvent_t> events;
  std::vector<std::string> names;
  int used = 0, cap = 0;
  bool armed = false;
};
thread_local TimingSession g_timing;
}  // namespace

namespace esm {
bool timing_slot(const char* kernel_name, hipEvent_t* start, hipEvent_t* stop) {
  TimingSession& t = g_timing;
  if (!t.armed || t.used >= t.cap) return false;
  *start = t.events[2 * t.used];
  *stop = t.events[2 * t.used + 1];
  std::string n(kernel_name);
  if (n.size() >= 2 && n.front() == '(' && n.back() == ')') n = n.substr(1, n.size() - 2);
  t.names[t.used++] = n;
  return true;
}
}  // namespace esm

extern "C" {

const char* esm_last_error(void) { return g_err.c_str(); }

const char* esm_version(void) { return "esmfold2_amd 0.2.0 gfx950"; }

const char* esm_source_hash(void) { return kSourceTag + 7; }

int tmu_leading_dim(int L) { return L <= 0 ? 0 : round_up(L, 8); }

// Halfs per channel of one workspace plane: the larger of [L, ld] and the fragment layout
// the fused forward's operands use.
static size_t tmu_plane_halfs(int L) {
  const size_t rows = (size_t)L * tmu_leading_dim(L), frag = esm::FragLayout::plane_halfs(L);
  return rows > frag ? rows : frag;
}

size_t tmu_workspace_bytes(int B, int L, int c) {
  if (B <= 0 || L <= 0 || c <= 0) return 0;
  const size_t plane = (size_t)B * c * tmu_plane_halfs(L) * sizeof(esm_half);
  const size_t a256 = (plane + 255) / 256 * 256;
  return (c == 128 ? 3 : 4) * a256;  // a, b, x (and the wide path's LN_in(z) plane)
}

// frag: write a, b in the fragment layout (the fused forward) instead of [B, c, L, ld].
static int project_impl(const esm_half* z, const esm_half* mask, const float* ln_w, const float* ln_b, float ln_eps,
                        const esm_half* w, esm_half* a_out, esm_half* b_out, int B, int L, int C, int c, int ld,
                        int incoming, bool frag, void* stream) {
  if (B < 0 || L < 0) return fail(ESM_ERR_SHAPE, "tmu_project: B=%d L=%d must be >= 0", B, L);
  if (C != 128 || c != 128) return fail(ESM_ERR_UNSUPPORTED, "tmu_project: C=%d c=%d (supported: 128, 128)", C, c);
  if (B == 0 || L == 0) return ok();
  if (!z || !ln_w || !ln_b || !w || !a_out || !b_out) return fail(ESM_ERR_NULL, "tmu_project: NULL pointer");
  if (L > kMaxL) return fail(ESM_ERR_SHAPE, "tmu_project: L=%d exceeds %d", L, kMaxL);
  if (ld % 8 != 0 || ld < L || ld > round_up(L, esm::kCellTile))
    return fail(ESM_ERR_SHAPE, "tmu_project: ld=%d must be a multiple of 8 in [L, roundup(L,%d)] (L=%d)", ld,
                esm::kCellTile, L);
  if (!aligned16(z) || !aligned16(w) || !aligned16(a_out) || !aligned16(b_out))
    return fail(ESM_ERR_ALIGN, "tmu_project: z, w, a, b must be 16-byte aligned");
  if (!(ln_eps >= 0.f)) return fail(ESM_ERR_SHAPE, "tmu_project: eps must be >= 0");
  esm::ProjectArgs a{H(z), mask ? H(mask) : nullptr, ln_w, ln_b, ln_eps, H(w), H(a_out), H(b_out), B, L, ld,
                     incoming ? 1 : 0, 0, 0};
  long long ntiles;
  if (frag) {  // blocks of 8 x 8 cells
    a.frag = 1;
    a.rbn = (L + 31) / 32;
    a.kbn = (L + 15) / 16;
    a.tiles_per_line = (L + 7) / 8;
    ntiles = (long long)B * a.tiles_per_line * a.tiles_per_line;
  } else {
    a.tiles_per_line = (L + esm::kCellTile - 1) / esm::kCellTile;
    ntiles = (long long)B * L * a.tiles_per_line;
  }
  if (ntiles > 0x7fffffffLL) return fail(ESM_ERR_SHAPE, "tmu_project: too many tiles");
  a.ntiles = (int)ntiles;
  const int grid = (int)(ntiles < cu_count() ? ntiles : cu_count());
  return hip_status(esm::launch_project(a, grid, (hipStream_t)stream), "tmu_project launch");
}

int tmu_project(const esm_half* z, const esm_half* mask, const float* ln_w, const float* ln_b, float ln_eps,
                const esm_half* w, esm_half* a_out, esm_half* b_out, int B, int L, int C, int c, int ld,
                int incoming, void* stream) {
  return project_impl(z, mask, ln_w, ln_b, ln_eps, w, a_out, b_out, B, L, C, c, ld, incoming, false, stream);
}

size_t tmu_frag_plane_elems(int L) { return L <= 0 ? 0 : esm::FragLayout::plane_halfs(L); }

int tmu_project_frag(const esm_half* z, const esm_half* mask, const float* ln_w, const float* ln_b, float ln_eps,
                     const esm_half* w, esm_half* a_out, esm_half* b_out, int B, int L, int C, int c,
                     int incoming, void* stream) {
  return project_impl(z, mask, ln_w, ln_b, ln_eps, w, a_out, b_out, B, L, C, c, tmu_leading_dim(L), incoming, true,
                      stream);
}

int tmu_contract_frag(const esm_half* a, const esm_half* b, esm_half* x, int batch, int L, int ldx, float scale,
                      void* stream) {
  if (batch < 0 || L < 0) return fail(ESM_ERR_SHAPE, "tmu_contract_frag: batch=%d L=%d must be >= 0", batch, L);
  if (batch == 0 || L == 0) return ok();
  if (!a || !b || !x) return fail(ESM_ERR_NULL, "tmu_contract_frag: NULL pointer");
  if (L > kMaxL || batch > 65535)
    return fail(ESM_ERR_SHAPE, "tmu_contract_frag: L=%d batch=%d out of range", L, batch);
  if (ldx % 8 != 0 || ldx < L || ldx > round_up(L, 32))
    return fail(ESM_ERR_SHAPE, "tmu_contract_frag: ldx=%d must be a multiple of 8 in [L, roundup(L, 32)] (L=%d)", ldx,
                L);
  if (!aligned16(a) || !aligned16(b) || !aligned16(x))
    return fail(ESM_ERR_ALIGN, "tmu_contract_frag: a, b, x must be 16-byte aligned");
  esm::ContractArgs args{H(a), H(b), H(x), batch, L, 0, ldx, scale, 1};
  return hip_status(esm::launch_contract(args, (hipStream_t)stream), "tmu_contract_frag launch");
}

int tmu_contract(const esm_half* a, const esm_half* b, esm_half* x, int batch, int L, int ld, int ldx, float scale,
                 void* stream) {
  if (batch < 0 || L < 0) return fail(ESM_ERR_SHAPE, "tmu_contract: batch=%d L=%d must be >= 0", batch, L);
  if (batch == 0 || L == 0) return ok();
  if (!a || !b || !x) return fail(ESM_ERR_NULL, "tmu_contract: NULL pointer");
  if (L > kMaxL || batch > 65535) return fail(ESM_ERR_SHAPE, "tmu_contract: L=%d batch=%d out of range", L, batch);
  // x columns [L, ldx) are written with zeros; the output blocks cover every column below
  // roundup(L, 64), so ldx may not exceed it.
  if (ld % 8 != 0 || ld < L || ldx % 8 != 0 || ldx < L || ldx > round_up(L, 64))
    return fail(ESM_ERR_SHAPE, "tmu_contract: ld=%d ldx=%d must be multiples of 8, >= L=%d, ldx <= %d", ld, ldx, L,
                round_up(L, 64));
  if (!aligned16(a) || !aligned16(b) || !aligned16(x))
    return fail(ESM_ERR_ALIGN, "tmu_contract: a, b, x must be 16-byte aligned");
  esm::ContractArgs args{H(a), H(b), H(x), batch, L, ld, ldx, scale};
  return hip_status(esm::launch_contract(args, (hipStream_t)stream), "tmu_contract launch");
}

int tmu_epilogue(const esm_half* x, int ldx, const esm_half* z, const esm_half* mask, const float* ln_in_w,
                 const float* ln_in_b, float ln_in_eps, const float* ln_mix_w, const float* ln_mix_b,
                 float ln_mix_eps, const esm_half* w_emit, const esm_half* w_gate, esm_half* out, int B, int L,
                 int C, int c, int residual, int out_mask, void* stream) {
  if (B < 0 || L < 0) return fail(ESM_ERR_SHAPE, "tmu_epilogue: B=%d L=%d must be >= 0", B, L);
  if (C != 128 || c != 128) return fail(ESM_ERR_UNSUPPORTED, "tmu_epilogue: C=%d c=%d (supported: 128, 128)", C, c);
  if (B == 0 || L == 0) return ok();
  if (!x || !z || !ln_in_w || !ln_in_b || !ln_mix_w || !ln_mix_b || !w_emit || !w_gate || !out)
    return fail(ESM_ERR_NULL, "tmu_epilogue: NULL pointer");
  if (L > kMaxL) return fail(ESM_ERR_SHAPE, "tmu_epilogue: L=%d exceeds %d", L, kMaxL);
  if (ldx % 8 != 0 || ldx < L) return fail(ESM_ERR_SHAPE, "tmu_epilogue: ldx=%d must be a multiple of 8, >= L", ldx);
  if (!aligned16(x) || !aligned16(z) || !aligned16(w_emit) || !aligned16(w_gate) || !aligned16(out))
    return fail(ESM_ERR_ALIGN, "tmu_epilogue: x, z, w_emit, w_gate, out must be 16-byte aligned");
  if (out == z && !residual)
    return fail(ESM_ERR_SHAPE, "tmu_epilogue: out may alias z only with residual=1");
  if (out_mask && !mask) return fail(ESM_ERR_NULL, "tmu_epilogue: out_mask=1 needs a mask");
  if (!(ln_in_eps >= 0.f) || !(ln_mix_eps >= 0.f)) return fail(ESM_ERR_SHAPE, "tmu_epilogue: eps must be >= 0");
  esm::EpilogueArgs e{H(x), ldx, H(z), mask ? H(mask) : nullptr, ln_in_w, ln_in_b, ln_in_eps, ln_mix_w, ln_mix_b,
                      ln_mix_eps, H(w_emit), H(w_gate), H(out), B, L, residual ? 1 : 0, out_mask ? 1 : 0, 0, 0};
  // units of 32 cells of one pair row, one per wave per round
  e.tiles_per_line = (L + esm::kEpiUnit - 1) / esm::kEpiUnit;
  const long long nunits = (long long)B * L * e.tiles_per_line;
  if (nunits > 0x7fffffffLL) return fail(ESM_ERR_SHAPE, "tmu_epilogue: too many units");
  e.ntiles = (int)nunits;
  const long long cap = cu_count();  // at most one persistent workgroup per CU
  const long long want = (nunits + esm::kEpiWaves - 1) / esm::kEpiWaves;
  const int grid = (int)(want < cap ? want : cap);
  return hip_status(esm::launch_epilogue(e, grid, (hipStream_t)stream), "tmu_epilogue launch");
}

// The wide path of tmu_forward (C = c, a multiple of 128 other than 128, up to 512): five
// launches in the workspace planes a | b | x | n (x / 256 as in the narrow path):
//   n = LN_in(z) (cell-major)  ->  a, b = gate(n W^T) (channel-major, GATE_CM)  ->  x = a b^T
//   ->  y = LN_mix(x) (cell-major, into plane a)  ->  out = [z +] (y W_e^T) * sigmoid(n W_g^T)
static int tmu_forward_wide(const esm_half* z, const esm_half* mask, const float* ln_in_w, const float* ln_in_b,
                            float ln_in_eps, const esm_half* w_bundle, const float* ln_mix_w, const float* ln_mix_b,
                            float ln_mix_eps, const esm_half* w_emit, const esm_half* w_gate, esm_half* out,
                            void* workspace, int B, int L, int C, int outgoing, int residual, int out_mask,
                            void* stream) {
  const int c = C;
  hipStream_t st = (hipStream_t)stream;
  const int ld = tmu_leading_dim(L);
  const size_t ncell = (size_t)B * L * L;
  const size_t plane = (size_t)B * c * tmu_plane_halfs(L);
  const size_t a256 = (plane * sizeof(esm_half) + 255) / 256 * 256 / sizeof(esm_half);
  half_t* wa = static_cast<half_t*>(workspace);
  half_t* wb = wa + a256;
  half_t* wx = wb + a256;
  half_t* wn = wx + a256;
  const float kScale = 1.0f / 256.0f;
  hipError_t e = esm::launch_ln_rows(z, nullptr, false, ln_in_w, ln_in_b, ln_in_eps, wn, ncell, C, st);
  if (e != hipSuccess) return hip_status(e, "tmu_forward ln_rows launch");
  esm::WideArgs g{};
  g.a1 = wn;
  g.w1 = H(w_bundle);                       // signal rows [s_a | s_b]
  g.w2 = H(w_bundle) + (size_t)2 * c * C;   // gate rows [g_a | g_b]
  g.K = C;
  g.N = 2 * c;
  g.B = B;
  g.L = L;
  g.tiles_per_line = (L + 127) / 128;
  g.transpose = outgoing ? 0 : 1;
  g.mask = mask ? H(mask) : nullptr;
  g.plane_a = wa;
  g.plane_b = wb;
  g.c = c;
  g.ld = ld;
  // K = C <= 256 runs the weight-stationary GEMM, which writes a, b in the fragment layout
  // (the contraction then reads each operand fragment straight into registers)
  const bool frag = C <= 256;
  if (frag) {
    g.frag = 1;
    g.rbn = (L + 31) / 32;
    g.kbn = (L + 15) / 16;
  }
  if (esm::wide_gemm_blocks(g) > 0x7fffffffLL) return fail(ESM_ERR_SHAPE, "tmu_forward: too many tiles");
  e = esm::launch_wide_gemm(g, esm::kWideGateCM, st, cu_count());
  if (e != hipSuccess) return hip_status(e, "tmu_forward gate launch");
  esm::ContractArgs ca{wa, wb, wx, B * c, L, ld, ld, kScale, frag ? 1 : 0};
  e = esm::launch_contract(ca, st);
  if (e != hipSuccess) return hip_status(e, "tmu_forward contract launch");
  e = esm::launch_ln_cf_to_cl(wx, ld, ln_mix_w, ln_mix_b, ln_mix_eps * kScale * kScale, wa, B, L, c, st);
  if (e != hipSuccess) return hip_status(e, "tmu_forward ln_cf_to_cl launch");
  esm::WideArgs r{};
  r.a1 = wa;                                // y = LN_mix(x), cell-major
  r.w1 = H(w_emit);
  r.a2 = wn;                                // n = LN_in(z)
  r.w2 = H(w_gate);
  r.K = C;
  r.N = C;
  r.B = B;
  r.L = L;
  r.tiles_per_line = (L + 127) / 128;
  r.out = H(out);
  r.ldo = C;
  r.z = H(z);
  r.residual = residual ? 1 : 0;
  r.mask = mask ? H(mask) : nullptr;
  r.out_mask = out_mask ? 1 : 0;
  e = esm::launch_wide_gemm(r, esm::kWideResGate, st, cu_count());
  return hip_status(e, "tmu_forward emit launch");
}

static bool wide_width(int C) { return C != 128 && C % 128 == 0 && C <= 512; }

int tmu_forward(const esm_half* z, const esm_half* mask, const float* ln_in_w, const float* ln_in_b, float ln_in_eps,
                const esm_half* w_bundle, const float* ln_mix_w, const float* ln_mix_b, float ln_mix_eps,
                const esm_half* w_emit, const esm_half* w_gate, esm_half* out, void* workspace, int B, int L, int C,
                int c, int outgoing, int residual, int out_mask, void* stream) {
  if (B < 0 || L < 0) return fail(ESM_ERR_SHAPE, "tmu_forward: B=%d L=%d must be >= 0", B, L);
  if (!((C == 128 && c == 128) || (C == c && wide_width(C))))
    return fail(ESM_ERR_UNSUPPORTED, "tmu_forward: C=%d c=%d (supported: C = c, 128 or a multiple of 128 up to 512)",
                C, c);
  if (B == 0 || L == 0) return ok();
  // everything is checked here, before the first of the launches
  if (!z || !ln_in_w || !ln_in_b || !w_bundle || !ln_mix_w || !ln_mix_b || !w_emit || !w_gate || !out)
    return fail(ESM_ERR_NULL, "tmu_forward: NULL pointer");
  if (!workspace) return fail(ESM_ERR_NULL, "tmu_forward: NULL workspace");
  if (L > kMaxL) return fail(ESM_ERR_SHAPE, "tmu_forward: L=%d exceeds %d", L, kMaxL);
  // No bound on B * L * L * C beyond memory: every kernel addresses its tile, line or channel
  // plane from a 64-bit base, so each 32-bit buffer offset stays below 2 GB for L <= kMaxL.
  if ((long long)B * c > 65535)
    return fail(ESM_ERR_SHAPE, "tmu_forward: B=%d c=%d: B*c must be <= 65535", B, c);
  if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0)
    return fail(ESM_ERR_ALIGN, "tmu_forward: workspace must be 256-byte aligned");
  if (!aligned16(z) || !aligned16(w_bundle) || !aligned16(w_emit) || !aligned16(w_gate) || !aligned16(out))
    return fail(ESM_ERR_ALIGN, "tmu_forward: z, weights and out must be 16-byte aligned");
  if (out == z && !residual) return fail(ESM_ERR_SHAPE, "tmu_forward: out may alias z only with residual=1");
  if (out_mask && !mask) return fail(ESM_ERR_NULL, "tmu_forward: out_mask=1 needs a mask");
  if (!(ln_in_eps >= 0.f) || !(ln_mix_eps >= 0.f)) return fail(ESM_ERR_SHAPE, "tmu_forward: eps must be >= 0");
  if (C != 128)
    return tmu_forward_wide(z, mask, ln_in_w, ln_in_b, ln_in_eps, w_bundle, ln_mix_w, ln_mix_b, ln_mix_eps, w_emit,
                            w_gate, out, workspace, B, L, C, outgoing, residual, out_mask, stream);
  const int ld = tmu_leading_dim(L);
  const size_t plane = (size_t)B * c * tmu_plane_halfs(L);
  const size_t a256 = (plane * sizeof(esm_half) + 255) / 256 * 256 / sizeof(esm_half);
  esm_half* wa = static_cast<esm_half*>(workspace);
  esm_half* wb = wa + a256;
  esm_half* wx = wb + a256;
  // fp16 range scheme (mlx_trunk.py:14-19): the contraction is stored as x/256
  // and norm_mix's eps divided by 256^2; LN(x/s, eps/s^2) == LN(x, eps) exactly.
  const float kScale = 1.0f / 256.0f;
  // a and b go through the workspace in the fragment layout: the contraction then loads
  // every operand fragment straight into registers (same bits as the [B, c, L, ld] path)
  int rc = project_impl(z, mask, ln_in_w, ln_in_b, ln_in_eps, w_bundle, wa, wb, B, L, C, c, ld, outgoing ? 0 : 1,
                        true, stream);
  if (rc) return rc;
  rc = tmu_contract_frag(wa, wb, wx, B * c, L, ld, kScale, stream);
  if (rc) return rc;
  return tmu_epilogue(wx, ld, z, mask, ln_in_w, ln_in_b, ln_in_eps, ln_mix_w, ln_mix_b, ln_mix_eps * kScale * kScale,
                      w_emit, w_gate, out, B, L, C, c, residual, out_mask, stream);
}

int tmu_pair_forward(const esm_half* z, const esm_half* mask, const float* o_ln_in_w, const float* o_ln_in_b,
                     float o_ln_in_eps, const esm_half* o_w_bundle, const float* o_ln_mix_w, const float* o_ln_mix_b,
                     float o_ln_mix_eps, const esm_half* o_w_emit, const esm_half* o_w_gate, int o_out_mask,
                     const float* i_ln_in_w, const float* i_ln_in_b, float i_ln_in_eps, const esm_half* i_w_bundle,
                     const float* i_ln_mix_w, const float* i_ln_mix_b, float i_ln_mix_eps, const esm_half* i_w_emit,
                     const esm_half* i_w_gate, int i_out_mask, esm_half* out, void* workspace, int B, int L, int C,
                     int c, void* stream) {
  // The incoming update's arguments are checked before the outgoing one launches: a bad
  // argument launches nothing. (Its z is out, which the first call writes.)
  if (B < 0 || L < 0) return fail(ESM_ERR_SHAPE, "tmu_pair_forward: B=%d L=%d must be >= 0", B, L);
  if (B > 0 && L > 0) {
    if (!i_ln_in_w || !i_ln_in_b || !i_w_bundle || !i_ln_mix_w || !i_ln_mix_b || !i_w_emit || !i_w_gate)
      return fail(ESM_ERR_NULL, "tmu_pair_forward: NULL pointer");
    if (!aligned16(i_w_bundle) || !aligned16(i_w_emit) || !aligned16(i_w_gate))
      return fail(ESM_ERR_ALIGN, "tmu_pair_forward: weights must be 16-byte aligned");
    if (i_out_mask && !mask) return fail(ESM_ERR_NULL, "tmu_pair_forward: out_mask=1 needs a mask");
    if (!(i_ln_in_eps >= 0.f) || !(i_ln_mix_eps >= 0.f))
      return fail(ESM_ERR_SHAPE, "tmu_pair_forward: eps must be >= 0");
  }
  int rc = tmu_forward(z, mask, o_ln_in_w, o_ln_in_b, o_ln_in_eps, o_w_bundle, o_ln_mix_w, o_ln_mix_b, o_ln_mix_eps,
                       o_w_emit, o_w_gate, out, workspace, B, L, C, c, 1, 1, o_out_mask, stream);
  if (rc) return rc;
  return tmu_forward(out, mask, i_ln_in_w, i_ln_in_b, i_ln_in_eps, i_w_bundle, i_ln_mix_w, i_ln_mix_b, i_ln_mix_eps,
                     i_w_emit, i_w_gate, out, workspace, B, L, C, c, 0, 1, i_out_mask, stream);
}

// The sized forms: a workspace smaller than tmu_workspace_bytes(B, L, c) is refused before
// anything else is looked at beyond the widths, so a buffer sized for another (B, L, c) or an
// older layout is an error, not an overrun.
static int tmu_ws_check(const char* fn, size_t have, int B, int L, int c) {
  if (B <= 0 || L <= 0 || c <= 0 || c > 512) return 0;  // the unsized entry point reports these
  const size_t need = tmu_workspace_bytes(B, L, c);
  if (have < need)
    return fail(ESM_ERR_SHAPE, "%s: workspace of %zu bytes, %zu needed for B=%d L=%d c=%d", fn, have, need, B, L, c);
  return 0;
}

int tmu_forward_ws(const esm_half* z, const esm_half* mask, const float* ln_in_w, const float* ln_in_b,
                   float ln_in_eps, const esm_half* w_bundle, const float* ln_mix_w, const float* ln_mix_b,
                   float ln_mix_eps, const esm_half* w_emit, const esm_half* w_gate, esm_half* out, void* workspace,
                   size_t workspace_bytes, int B, int L, int C, int c, int outgoing, int residual, int out_mask,
                   void* stream) {
  if (const int rc = tmu_ws_check("tmu_forward_ws", workspace_bytes, B, L, c)) return rc;
  return tmu_forward(z, mask, ln_in_w, ln_in_b, ln_in_eps, w_bundle, ln_mix_w, ln_mix_b, ln_mix_eps, w_emit, w_gate,
                     out, workspace, B, L, C, c, outgoing, residual, out_mask, stream);
}

int tmu_pair_forward_ws(const esm_half* z, const esm_half* mask, const float* o_ln_in_w, const float* o_ln_in_b,
                        float o_ln_in_eps, const esm_half* o_w_bundle, const float* o_ln_mix_w,
                        const float* o_ln_mix_b, float o_ln_mix_eps, const esm_half* o_w_emit,
                        const esm_half* o_w_gate, int o_out_mask, const float* i_ln_in_w, const float* i_ln_in_b,
                        float i_ln_in_eps, const esm_half* i_w_bundle, const float* i_ln_mix_w,
                        const float* i_ln_mix_b, float i_ln_mix_eps, const esm_half* i_w_emit,
                        const esm_half* i_w_gate, int i_out_mask, esm_half* out, void* workspace,
                        size_t workspace_bytes, int B, int L, int C, int c, void* stream) {
  if (const int rc = tmu_ws_check("tmu_pair_forward_ws", workspace_bytes, B, L, c)) return rc;
  return tmu_pair_forward(z, mask, o_ln_in_w, o_ln_in_b, o_ln_in_eps, o_w_bundle, o_ln_mix_w, o_ln_mix_b,
                          o_ln_mix_eps, o_w_emit, o_w_gate, o_out_mask, i_ln_in_w, i_ln_in_b, i_ln_in_eps, i_w_bundle,
                          i_ln_mix_w, i_ln_mix_b, i_ln_mix_eps, i_w_emit, i_w_gate, i_out_mask, out, workspace, B, L,
                          C, c, stream);
}

// Checks shared by the q8 GEMM entry points (fn names the caller in the messages); out is
// y (8-byte aligned) or the partials (256-byte aligned). Sets *empty for a no-op shape.
// With packed codes (qp) the weights are qp and sb, and q, s, b are not read.
static int q8_check_weights(const char* fn, const esm_half* x, const uint8_t* q, const esm_half* s, const esm_half* b,
                            const uint32_t* sb, const uint8_t* qp, const void* out, unsigned out_align, int M, int K,
                            int N, int group, bool* empty);
static int q8_check(const char* fn, const esm_half* x, const uint8_t* q, const esm_half* s, const esm_half* b,
                    const void* out, unsigned out_align, int M, int K, int N, int group, bool* empty) {
  return q8_check_weights(fn, x, q, s, b, nullptr, nullptr, out, out_align, M, K, N, group, empty);
}
static int q8_check_weights(const char* fn, const esm_half* x, const uint8_t* q, const esm_half* s, const esm_half* b,
                            const uint32_t* sb, const uint8_t* qp, const void* out, unsigned out_align, int M, int K,
                            int N, int group, bool* empty) {
  *empty = false;
  if (M < 0 || K < 0 || N < 0) return fail(ESM_ERR_SHAPE, "%s: M=%d K=%d N=%d must be >= 0", fn, M, K, N);
  if (group != 64) return fail(ESM_ERR_UNSUPPORTED, "%s: group=%d (supported: 64)", fn, group);
  if (M == 0 || N == 0) {
    *empty = true;
    return ok();
  }
  if (K == 0 || K % 64 != 0 || N % 64 != 0)
    return fail(ESM_ERR_SHAPE, "%s: K=%d and N=%d must be positive multiples of 64", fn, K, N);
  if (K > kQ8MaxK) return fail(ESM_ERR_SHAPE, "%s: K=%d too large (max %d)", fn, K, kQ8MaxK);
  if ((long long)N * K >= (1LL << 31) || (long long)M * K * 2 >= (1LL << 31))
    return fail(ESM_ERR_SHAPE, "%s: M=%d, K=%d, N=%d: x or q exceeds 2 GB", fn, M, K, N);
  if (qp) {
    if (!x || !sb || !out) return fail(ESM_ERR_NULL, "%s: NULL pointer", fn);
    if (!aligned16(x) || !aligned16(qp) || !aligned16(sb) || (reinterpret_cast<uintptr_t>(out) & (out_align - 1)) != 0)
      return fail(ESM_ERR_ALIGN, "%s: x, qp, sb must be 16-byte aligned and the output %u-byte aligned", fn,
                  out_align);
    return ok();
  }
  if (!x || !q || !s || !b || !out) return fail(ESM_ERR_NULL, "%s: NULL pointer", fn);
  if (!aligned16(x) || !aligned16(q) || (reinterpret_cast<uintptr_t>(out) & (out_align - 1)) != 0 ||
      (reinterpret_cast<uintptr_t>(s) & 1u) != 0 || (reinterpret_cast<uintptr_t>(b) & 1u) != 0)
    return fail(ESM_ERR_ALIGN, "%s: x, q must be 16-byte aligned and the output %u-byte aligned", fn, out_align);
  return ok();
}

int q8_linear_ws(const esm_half* x, const uint8_t* q, const esm_half* s, const esm_half* b, const uint32_t* sb,
                 esm_half* y, int M, int K, int N, int group, void* workspace, size_t workspace_bytes, void* stream) {
  bool empty;
  if (const int rc = q8_check("q8_linear", x, q, s, b, y, 8, M, K, N, group, &empty)) return rc;
  if (empty) return ok();
  Q8Plan pl = q8_plan(M, K, N);
  if ((long long)pl.mtiles * pl.ntiles * pl.splits > 0x7fffffffLL)
    return fail(ESM_ERR_SHAPE, "q8_linear: M=%d N=%d too large", M, N);
  if (!workspace) {
    pl.splits = 1;  // no workspace: one workgroup per tile, no partials
  } else if (pl.splits > 1) {
    if (workspace_bytes < pl.bytes)
      return fail(ESM_ERR_SHAPE, "q8_linear: workspace of %zu bytes, %zu needed", workspace_bytes, pl.bytes);
    if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0)
      return fail(ESM_ERR_ALIGN, "q8_linear: workspace must be 256-byte aligned");
  }
  if (sb && !aligned16(sb)) return fail(ESM_ERR_ALIGN, "q8_linear: packed scales must be 16-byte aligned");
  esm::Q8Args a{H(x), q, H(s), H(b), H(y), M, K, N, pl.mtiles, pl.ntiles, pl.splits,
                pl.splits > 1 ? static_cast<float*>(workspace) : nullptr, sb, nullptr, 0, pl.nb};
  return hip_status(esm::launch_q8_linear(a, (hipStream_t)stream), "q8_linear launch");
}

int q8_linear_noalloc(const esm_half* x, const uint8_t* q, const esm_half* s, const esm_half* b, const uint32_t* sb,
                      esm_half* y, int M, int K, int N, int group, void* stream) {
  static_assert(esm::kQ8ScratchBytes == ESM_Q8_NOALLOC_SCRATCH_BYTES, "header and library agree on the scratch");
  bool empty;
  if (const int rc = q8_check("q8_linear_noalloc", x, q, s, b, y, 8, M, K, N, group, &empty)) return rc;
  if (empty) return ok();
  const Q8Plan pl = q8_plan(M, K, N);
  if ((long long)pl.mtiles * pl.ntiles * pl.splits > 0x7fffffffLL)
    return fail(ESM_ERR_SHAPE, "q8_linear_noalloc: M=%d N=%d too large", M, N);
  if (pl.splits > 1 && pl.bytes > esm::kQ8ScratchBytes)
    return fail(ESM_ERR_SHAPE, "q8_linear_noalloc: M=%d K=%d N=%d needs %zu bytes of split-K scratch, the static "
                "scratch holds %zu", M, K, N, pl.bytes, esm::kQ8ScratchBytes);
  if (sb && !aligned16(sb)) return fail(ESM_ERR_ALIGN, "q8_linear_noalloc: packed scales must be 16-byte aligned");
  float* part = nullptr;
  if (pl.splits > 1) {
    const hipError_t e = esm::q8_scratch_address(&part);
    if (e != hipSuccess) return hip_status(e, "q8_linear_noalloc: scratch address");
  }
  esm::Q8Args a{H(x), q, H(s), H(b), H(y), M, K, N, pl.mtiles, pl.ntiles, pl.splits, part, sb, nullptr, 0, pl.nb};
  return hip_status(esm::launch_q8_linear(a, (hipStream_t)stream), "q8_linear_noalloc launch");
}

size_t q8_linear_partials_bytes(int M, int K, int N) {
  if (M <= 0 || K <= 0 || N <= 0 || K % 64 != 0 || N % 64 != 0 || K > kQ8MaxK) return 0;
  return q8_plan(M, K, N).bytes;
}

int q8_linear_partials(const esm_half* x, const uint8_t* q, const esm_half* s, const esm_half* b, const uint32_t* sb,
                       float* parts, size_t parts_bytes, int* splits, int M, int K, int N, int group, void* stream) {
  bool empty;
  if (!splits) return fail(ESM_ERR_NULL, "q8_linear_partials: NULL splits");
  *splits = 0;
  if (const int rc = q8_check("q8_linear_partials", x, q, s, b, parts, 256, M, K, N, group, &empty)) return rc;
  if (empty) return ok();
  const Q8Plan pl = q8_plan(M, K, N);
  if ((long long)pl.mtiles * pl.ntiles * pl.splits > 0x7fffffffLL)
    return fail(ESM_ERR_SHAPE, "q8_linear_partials: M=%d N=%d too large", M, N);
  if (parts_bytes < pl.bytes)
    return fail(ESM_ERR_SHAPE, "q8_linear_partials: %zu bytes for the partials, %zu needed", parts_bytes, pl.bytes);
  if (sb && !aligned16(sb)) return fail(ESM_ERR_ALIGN, "q8_linear_partials: packed scales must be 16-byte aligned");
  *splits = pl.splits;
  esm::Q8Args a{H(x), q, H(s), H(b), nullptr, M, K, N, pl.mtiles, pl.ntiles, pl.splits, parts, sb, nullptr, 0, pl.nb};
  return hip_status(esm::launch_q8_linear(a, (hipStream_t)stream), "q8_linear_partials launch");
}

int q8_linear_packed_ws(const esm_half* x, const uint8_t* qp, const uint32_t* sb, esm_half* y, int M, int K, int N,
                        int group, void* workspace, size_t workspace_bytes, void* stream) {
  bool empty;
  if (!qp) return fail(ESM_ERR_NULL, "q8_linear_packed_ws: NULL packed codes");
  if (const int rc = q8_check_weights("q8_linear_packed_ws", x, nullptr, nullptr, nullptr, sb, qp, y, 8, M, K, N, group,
                                      &empty))
    return rc;
  if (empty) return ok();
  Q8Plan pl = q8_plan(M, K, N);
  if ((long long)pl.mtiles * pl.ntiles * pl.splits > 0x7fffffffLL)
    return fail(ESM_ERR_SHAPE, "q8_linear_packed_ws: M=%d N=%d too large", M, N);
  if (!workspace) {
    pl.splits = 1;
  } else if (pl.splits > 1) {
    if (workspace_bytes < pl.bytes)
      return fail(ESM_ERR_SHAPE, "q8_linear_packed_ws: workspace of %zu bytes, %zu needed", workspace_bytes, pl.bytes);
    if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0)
      return fail(ESM_ERR_ALIGN, "q8_linear_packed_ws: workspace must be 256-byte aligned");
  }
  esm::Q8Args a{H(x), nullptr, nullptr, nullptr, H(y), M, K, N, pl.mtiles, pl.ntiles, pl.splits,
                pl.splits > 1 ? static_cast<float*>(workspace) : nullptr, sb, qp, 0, pl.nb};
  return hip_status(esm::launch_q8_linear(a, (hipStream_t)stream), "q8_linear_packed_ws launch");
}

int q8_linear_swiglu_packed_ws(const esm_half* x, const uint8_t* qp, const uint32_t* sb, esm_half* y, int M, int K,
                               int N, int group, void* workspace, size_t workspace_bytes, void* stream) {
  bool empty;
  if (!qp) return fail(ESM_ERR_NULL, "q8_linear_swiglu_packed_ws: NULL packed codes");
  if (const int rc = q8_check_weights("q8_linear_swiglu_packed_ws", x, nullptr, nullptr, nullptr, sb, qp, y, 8, M, K,
                                      N, group, &empty))
    return rc;
  if (empty) return ok();
  if (N % (2 * esm::kQ8SwigluHalf) != 0)
    return fail(ESM_ERR_SHAPE, "q8_linear_swiglu_packed_ws: N=%d must be a multiple of %d (SwiGLU pair tiles)", N,
                2 * esm::kQ8SwigluHalf);
  Q8Plan pl = q8_plan(M, K, N, true);
  if ((long long)pl.mtiles * pl.ntiles * pl.splits > 0x7fffffffLL)
    return fail(ESM_ERR_SHAPE, "q8_linear_swiglu_packed_ws: M=%d N=%d too large", M, N);
  if (!workspace) {
    pl.splits = 1;
  } else if (pl.splits > 1) {
    if (workspace_bytes < pl.bytes)
      return fail(ESM_ERR_SHAPE, "q8_linear_swiglu_packed_ws: workspace of %zu bytes, %zu needed", workspace_bytes,
                  pl.bytes);
    if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0)
      return fail(ESM_ERR_ALIGN, "q8_linear_swiglu_packed_ws: workspace must be 256-byte aligned");
  }
  esm::Q8Args a{H(x), nullptr, nullptr, nullptr, H(y), M, K, N, pl.mtiles, pl.ntiles, pl.splits,
                pl.splits > 1 ? static_cast<float*>(workspace) : nullptr, sb, qp, 1, pl.nb};
  return hip_status(esm::launch_q8_linear(a, (hipStream_t)stream), "q8_linear_swiglu_packed_ws launch");
}

int q8_linear_packed_partials(const esm_half* x, const uint8_t* qp, const uint32_t* sb, float* parts,
                              size_t parts_bytes, int* splits, int M, int K, int N, int group, void* stream) {
  bool empty;
  if (!splits) return fail(ESM_ERR_NULL, "q8_linear_packed_partials: NULL splits");
  *splits = 0;
  if (!qp) return fail(ESM_ERR_NULL, "q8_linear_packed_partials: NULL packed codes");
  if (const int rc = q8_check_weights("q8_linear_packed_partials", x, nullptr, nullptr, nullptr, sb, qp, parts, 256, M,
                                      K, N, group, &empty))
    return rc;
  if (empty) return ok();
  const Q8Plan pl = q8_plan(M, K, N);
  if ((long long)pl.mtiles * pl.ntiles * pl.splits > 0x7fffffffLL)
    return fail(ESM_ERR_SHAPE, "q8_linear_packed_partials: M=%d N=%d too large", M, N);
  if (parts_bytes < pl.bytes)
    return fail(ESM_ERR_SHAPE, "q8_linear_packed_partials: %zu bytes for the partials, %zu needed", parts_bytes,
                pl.bytes);
  *splits = pl.splits;
  esm::Q8Args a{H(x), nullptr, nullptr, nullptr, nullptr, M, K, N, pl.mtiles, pl.ntiles, pl.splits, parts, sb, qp, 0, pl.nb};
  return hip_status(esm::launch_q8_linear(a, (hipStream_t)stream), "q8_linear_packed_partials launch");
}

int q8_linear(const esm_half* x, const uint8_t* q, const esm_half* s, const esm_half* b, esm_half* y, int M, int K,
              int N, int group, void* stream) {
  return q8_linear_ws(x, q, s, b, nullptr, y, M, K, N, group, nullptr, 0, stream);
}

// The register-resident transition kernel covers C = 128 with ReLU at H in {256, 512} and
// SwiGLU at H = 256; every other shape runs the wide path (LayerNorm, then one GEMM with the
// activation fused, then one with the residual fused), whose hidden activations [cells, H]
// and LayerNormed input [cells, C] live in the caller's workspace.
static bool narrow_transition(int C, int H, bool swiglu) {
  return C == 128 && (swiglu ? H == 256 : (H == 256 || H == 512));
}

size_t pair_transition_workspace_bytes(int B, int L, int C, int hidden, int swiglu) {
  if (B <= 0 || L <= 0 || C <= 0 || hidden <= 0 || narrow_transition(C, hidden, swiglu != 0)) return 0;
  const size_t cells = (size_t)B * L * L;
  const auto al = [](size_t bytes) { return (bytes + 255) / 256 * 256; };
  return al(cells * C * sizeof(esm_half)) + al(cells * hidden * sizeof(esm_half));
}

int pair_transition_ws(const esm_half* z, esm_half* out, const float* ln_w, const float* ln_b, float eps,
                       const esm_half* w1, const esm_half* w2, const esm_half* w3, int B, int L, int C, int hidden,
                       void* workspace, size_t workspace_bytes, void* stream) {
  if (B < 0 || L < 0) return fail(ESM_ERR_SHAPE, "pair_transition: B=%d L=%d must be >= 0", B, L);
  const bool narrow = narrow_transition(C, hidden, w2 != nullptr);
  if (!narrow && !((C == 128 || wide_width(C)) && hidden > 0 && hidden % 32 == 0))
    return fail(ESM_ERR_UNSUPPORTED,
                "pair_transition: C=%d H=%d (supported: C a multiple of 128 up to 512, H a multiple of 32)", C, hidden);
  if (!(eps >= 0.f)) return fail(ESM_ERR_SHAPE, "pair_transition: eps must be >= 0");
  if (B == 0 || L == 0) return ok();
  if (L > kMaxL) return fail(ESM_ERR_SHAPE, "pair_transition: L=%d exceeds %d", L, kMaxL);
  const size_t ncells = (size_t)B * L * L;
  if (ncells / 32 > 0x7fffffffull) return fail(ESM_ERR_SHAPE, "pair_transition: B*L*L=%zu cells", ncells);
  if (!z || !out || !ln_w || !ln_b || !w1 || !w3) return fail(ESM_ERR_NULL, "pair_transition: NULL pointer");
  if (!aligned16(z) || !aligned16(out) || !aligned16(w1) || !aligned16(w3) || (w2 && !aligned16(w2)))
    return fail(ESM_ERR_ALIGN, "pair_transition: z, out, w1, w2, w3 must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  if (narrow) {
    esm::TransitionArgs a{H(z), H(out), ln_w, ln_b, eps, H(w1), w2 ? H(w2) : nullptr, H(w3), ncells, 0, hidden};
    const size_t ntiles = (ncells + 31) / 32;
    a.ntiles = (int)ntiles;
    const int grid = (int)(ntiles < (size_t)cu_count() ? ntiles : cu_count());
    return hip_status(esm::launch_transition(a, grid, st), "pair_transition launch");
  }
  const size_t need = pair_transition_workspace_bytes(B, L, C, hidden, w2 != nullptr);
  if (!workspace) return fail(ESM_ERR_NULL, "pair_transition: C=%d H=%d needs a workspace of %zu bytes", C, hidden, need);
  if (workspace_bytes < need)
    return fail(ESM_ERR_SHAPE, "pair_transition: workspace of %zu bytes, %zu needed", workspace_bytes, need);
  if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0)
    return fail(ESM_ERR_ALIGN, "pair_transition: workspace must be 256-byte aligned");
  half_t* wn = static_cast<half_t*>(workspace);
  half_t* wh = wn + (ncells * C * sizeof(esm_half) + 255) / 256 * 256 / sizeof(esm_half);
  hipError_t e = esm::launch_ln_rows(z, nullptr, false, ln_w, ln_b, eps, wn, ncells, C, st);
  if (e != hipSuccess) return hip_status(e, "pair_transition ln_rows launch");
  esm::WideArgs g{};
  g.a1 = wn;
  g.w1 = H(w1);
  g.w2 = w2 ? H(w2) : nullptr;
  g.K = C;
  g.N = hidden;
  g.B = B;
  g.L = L;
  g.tiles_per_line = (L + 127) / 128;
  g.out = wh;
  g.ldo = hidden;
  if (esm::wide_gemm_blocks(g) > 0x7fffffffLL) return fail(ESM_ERR_SHAPE, "pair_transition: too many tiles");
  e = esm::launch_wide_gemm(g, w2 ? esm::kWideSwiglu : esm::kWideRelu, st, cu_count());
  if (e != hipSuccess) return hip_status(e, "pair_transition hidden launch");
  esm::WideArgs r{};
  r.a1 = wh;
  r.w1 = H(w3);
  r.K = hidden;
  r.N = C;
  r.B = B;
  r.L = L;
  r.tiles_per_line = (L + 127) / 128;
  r.out = H(out);
  r.ldo = C;
  r.z = H(z);
  e = esm::launch_wide_gemm(r, esm::kWideResid, st, cu_count());
  return hip_status(e, "pair_transition output launch");
}

int pair_transition(const esm_half* z, esm_half* out, const float* ln_w, const float* ln_b, float eps,
                    const esm_half* w1, const esm_half* w2, const esm_half* w3, int B, int L, int C, int hidden,
                    void* stream) {
  return pair_transition_ws(z, out, ln_w, ln_b, eps, w1, w2, w3, B, L, C, hidden, nullptr, 0, stream);
}

// esmc_layer_norm and esmc_layer_norm_parts: y (fp16) or yp (fp32 partials of y), or neither.
static int esmc_ln_run(const char* fn, const float* x, const esm_half* y, const float* yp, int splits, float alpha,
                       float* x_out, const float* w, const float* b, float eps, esm_half* h, float* h_fp32, int M,
                       int D, void* stream) {
  if (M < 0 || D <= 0) return fail(ESM_ERR_SHAPE, "%s: M=%d D=%d", fn, M, D);
  if (D % 8 != 0 || D > 8192) return fail(ESM_ERR_UNSUPPORTED, "%s: D=%d (multiple of 8, <= 8192)", fn, D);
  if (!(eps >= 0.f)) return fail(ESM_ERR_SHAPE, "%s: eps must be >= 0", fn);
  if (yp && splits < 1) return fail(ESM_ERR_SHAPE, "%s: splits=%d must be >= 1", fn, splits);
  if (M == 0) return ok();
  const bool add = y || yp;
  if (!x || !w || (!h == !h_fp32) || (add && !x_out))
    return fail(ESM_ERR_NULL, "%s: NULL pointer (exactly one of h, h_fp32 is written)", fn);
  if (!aligned16(x) || (h && !aligned16(h)) || (h_fp32 && !aligned16(h_fp32)) || (y && !aligned16(y)) ||
      (yp && !aligned16(yp)) || (add && !aligned16(x_out)))
    return fail(ESM_ERR_ALIGN, "%s: x, y, x_out, h, h_fp32 must be 16-byte aligned", fn);
  esm::EsmcLnArgs a{x, y ? H(y) : nullptr, yp, yp ? splits : 0, alpha, x_out, w, b, eps, h ? H(h) : nullptr, h_fp32,
                    M, D};
  return hip_status(esm::launch_esmc_ln(a, (hipStream_t)stream), "esmc_layer_norm launch");
}

int esmc_layer_norm(const float* x, const esm_half* y, float alpha, float* x_out, const float* w, const float* b,
                    float eps, esm_half* h, float* h_fp32, int M, int D, void* stream) {
  return esmc_ln_run("esmc_layer_norm", x, y, nullptr, 0, alpha, x_out, w, b, eps, h, h_fp32, M, D, stream);
}

int esmc_layer_norm_parts(const float* x, const float* y_parts, int splits, float alpha, float* x_out, const float* w,
                          const float* b, float eps, esm_half* h, float* h_fp32, int M, int D, void* stream) {
  if (!y_parts && M > 0) return fail(ESM_ERR_NULL, "esmc_layer_norm_parts: NULL partials");
  return esmc_ln_run("esmc_layer_norm_parts", x, nullptr, y_parts, splits, alpha, x_out, w, b, eps, h, h_fp32, M, D,
                     stream);
}

int esmc_qk_rope(const esm_half* qkv, const float* q_ln, const float* k_ln, float eps, esm_half* q, esm_half* k,
                 esm_half* v, int B, int L, int n_heads, int head_dim, float rope_base, void* stream) {
  if (B < 0 || L < 0 || n_heads <= 0) return fail(ESM_ERR_SHAPE, "esmc_qk_rope: B=%d L=%d heads=%d", B, L, n_heads);
  if (head_dim != 64 || n_heads * 64 > 4096)
    return fail(ESM_ERR_UNSUPPORTED, "esmc_qk_rope: head_dim=%d heads=%d (head_dim 64, width <= 4096)", head_dim,
                n_heads);
  if (!(eps >= 0.f)) return fail(ESM_ERR_SHAPE, "esmc_qk_rope: eps must be >= 0");
  if (B == 0 || L == 0) return ok();
  if (!qkv || !q_ln || !k_ln || !q || !k || !v) return fail(ESM_ERR_NULL, "esmc_qk_rope: NULL pointer");
  if (!aligned16(qkv) || !aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(q_ln) || !aligned16(k_ln))
    return fail(ESM_ERR_ALIGN, "esmc_qk_rope: qkv, q_ln, k_ln, q, k, v must be 16-byte aligned");
  esm::EsmcRopeArgs a{H(qkv), q_ln, k_ln, eps, H(q), H(k), H(v), B, L, n_heads, std::log2(rope_base)};
  return hip_status(esm::launch_esmc_qk_rope(a, (hipStream_t)stream), "esmc_qk_rope launch");
}

int esmc_attention(const esm_half* q, const esm_half* k, const esm_half* v, const int* sequence_id, esm_half* o, int B,
                   int L, int n_heads, int head_dim, float scale, void* stream) {
  if (B < 0 || L < 0 || n_heads <= 0) return fail(ESM_ERR_SHAPE, "esmc_attention: B=%d L=%d heads=%d", B, L, n_heads);
  if (head_dim != 64 || L > 65536)
    return fail(ESM_ERR_UNSUPPORTED, "esmc_attention: head_dim=%d L=%d (64, L <= 65536)", head_dim, L);
  if (B == 0 || L == 0) return ok();
  if ((long long)B * n_heads > 65535) return fail(ESM_ERR_SHAPE, "esmc_attention: B*heads=%d too large", B * n_heads);
  if (!q || !k || !v || !o) return fail(ESM_ERR_NULL, "esmc_attention: NULL pointer");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || (reinterpret_cast<uintptr_t>(o) & 7u))
    return fail(ESM_ERR_ALIGN, "esmc_attention: q, k, v must be 16-byte and o 8-byte aligned");
  esm::EsmcAttnArgs a{H(q), H(k), H(v), sequence_id, H(o), B, L, n_heads, scale * 1.4426950408889634f};
  return hip_status(esm::launch_esmc_attention(a, (hipStream_t)stream), "esmc_attention launch");
}

int esmc_swiglu(const esm_half* x12, esm_half* y, int M, int F, void* stream) {
  if (M < 0 || F <= 0 || F % 8 != 0) return fail(ESM_ERR_SHAPE, "esmc_swiglu: M=%d F=%d (F multiple of 8)", M, F);
  if (M == 0) return ok();
  if (!x12 || !y) return fail(ESM_ERR_NULL, "esmc_swiglu: NULL pointer");
  if (!aligned16(x12) || !aligned16(y)) return fail(ESM_ERR_ALIGN, "esmc_swiglu: x12, y must be 16-byte aligned");
  return hip_status(esm::launch_esmc_swiglu(H(x12), H(y), (size_t)M, F, (hipStream_t)stream), "esmc_swiglu launch");
}

int parcae_step(const float* z, const float* z_init, const float* refined, const float* ln_w, const float* ln_b,
                float eps, const float* a, const esm_half* b_mat, float* z_out, int B, int L, int C, void* stream) {
  if (B < 0 || L < 0) return fail(ESM_ERR_SHAPE, "parcae_step: B=%d L=%d must be >= 0", B, L);
  if (C != 128 && C != 256) return fail(ESM_ERR_UNSUPPORTED, "parcae_step: C=%d (supported: 128, 256)", C);
  if (!(eps >= 0.f)) return fail(ESM_ERR_SHAPE, "parcae_step: eps must be >= 0");
  if (B == 0 || L == 0) return ok();
  const size_t ncells = (size_t)B * L * L;
  if (ncells * C * 4 >= (1ull << 31)) return fail(ESM_ERR_SHAPE, "parcae_step: B*L*L=%zu cells exceed 2 GB", ncells);
  if (!z || !z_init || !refined || !ln_w || !ln_b || !a || !b_mat || !z_out)
    return fail(ESM_ERR_NULL, "parcae_step: NULL pointer");
  if (!aligned16(z) || !aligned16(z_init) || !aligned16(refined) || !aligned16(z_out) || !aligned16(b_mat))
    return fail(ESM_ERR_ALIGN, "parcae_step: z, z_init, refined, z_out, b_mat must be 16-byte aligned");
  const size_t ntiles = (ncells + 31) / 32;
  esm::ParcaeArgs args{z, z_init, refined, ln_w, ln_b, eps, a, H(b_mat), z_out, ncells, (int)ntiles, C};
  // two workgroups per CU at C = 128 (20.1 against 21.7 us at L=238); at C = 256 one (45 us; two: 50)
  const size_t cap = (size_t)cu_count() * (C == 128 ? 2 : 1);
  const int grid = (int)(ntiles < cap ? ntiles : cap);
  return hip_status(esm::launch_parcae_step(args, grid, (hipStream_t)stream), "parcae_step launch");
}

int distogram_expected_distance(const float* r, const esm_half* w, const float* bias, const float* centers, float* ed,
                                int B, int L, int C, int nbins, void* stream) {
  if (B < 0 || L < 0) return fail(ESM_ERR_SHAPE, "distogram_expected_distance: B=%d L=%d", B, L);
  if ((C != 128 && C != 256) || (nbins != 64 && nbins != 128))
    return fail(ESM_ERR_UNSUPPORTED, "distogram_expected_distance: C=%d nbins=%d (C 128 or 256; 64 or 128 bins)", C,
                nbins);
  if (B == 0 || L == 0) return ok();
  if (L > kMaxL) return fail(ESM_ERR_SHAPE, "distogram_expected_distance: L=%d exceeds %d", L, kMaxL);
  if (!r || !w || !bias || !centers || !ed) return fail(ESM_ERR_NULL, "distogram_expected_distance: NULL pointer");
  if (!aligned16(r) || !aligned16(w)) return fail(ESM_ERR_ALIGN, "distogram_expected_distance: r, w must be 16-byte aligned");
  esm::DistoArgs args{r, H(w), bias, centers, ed, B, L, nbins, C};
  long long units = 0;  // one wave per 32 pairs j >= i of a row, 4 waves per workgroup
  for (int I = 0, JT = (L + 31) / 32; I < JT; I++) units += (long long)std::min(32, L - 32 * I) * (JT - I);
  const long long blocks = (B * units + 3) / 4;
  const int grid = (int)(blocks < 4LL * cu_count() ? blocks : 4LL * cu_count());
  return hip_status(esm::launch_expected_distance(args, grid, (hipStream_t)stream), "distogram_expected_distance launch");
}

int abs_diff_quantile(const float* x, const float* y, size_t n, float q, float* out, void* stream) {
  if (n == 0) return fail(ESM_ERR_SHAPE, "abs_diff_quantile: n must be >= 1");
  if (!(q >= 0.f && q <= 1.f)) return fail(ESM_ERR_SHAPE, "abs_diff_quantile: q=%g outside [0, 1]", (double)q);
  if (!x || !out) return fail(ESM_ERR_NULL, "abs_diff_quantile: NULL pointer");
  return hip_status(esm::launch_abs_diff_quantile(x, y, n, q, out, (hipStream_t)stream), "abs_diff_quantile launch");
}

size_t q8_packed_scales_bytes(int N, int K) {
  if (N <= 0 || K <= 0 || K % 64 != 0) return 0;
  return esm::q8_packed_scales_words(N, K) * sizeof(uint32_t);
}

int q8_pack_scales(const esm_half* s, const esm_half* b, uint32_t* sb, int N, int K, int group, void* stream) {
  if (N < 0 || K < 0) return fail(ESM_ERR_SHAPE, "q8_pack_scales: N=%d K=%d must be >= 0", N, K);
  if (group != 64) return fail(ESM_ERR_UNSUPPORTED, "q8_pack_scales: group=%d (supported: 64)", group);
  if (N == 0 || K == 0) return ok();
  if (K % 64 != 0) return fail(ESM_ERR_SHAPE, "q8_pack_scales: K=%d must be a multiple of 64", K);
  if (!s || !b || !sb) return fail(ESM_ERR_NULL, "q8_pack_scales: NULL pointer");
  if ((reinterpret_cast<uintptr_t>(s) & 1u) || (reinterpret_cast<uintptr_t>(b) & 1u) || !aligned16(sb))
    return fail(ESM_ERR_ALIGN, "q8_pack_scales: s, b must be 2-byte and sb 16-byte aligned");
  return hip_status(esm::launch_q8_pack(H(s), H(b), sb, N, K, (hipStream_t)stream), "q8_pack_scales launch");
}

size_t q8_packed_codes_bytes(int N, int K) {
  if (N <= 0 || K <= 0 || K % 64 != 0 || K > kQ8MaxK || (long long)N * K >= (1LL << 31)) return 0;
  return esm::q8_packed_codes_size(N, K);
}

int q8_pack_codes(const uint8_t* q, uint8_t* qp, int N, int K, int group, void* stream) {
  if (N < 0 || K < 0) return fail(ESM_ERR_SHAPE, "q8_pack_codes: N=%d K=%d must be >= 0", N, K);
  if (group != 64) return fail(ESM_ERR_UNSUPPORTED, "q8_pack_codes: group=%d (supported: 64)", group);
  if (N == 0 || K == 0) return ok();
  if (K % 64 != 0) return fail(ESM_ERR_SHAPE, "q8_pack_codes: K=%d must be a multiple of 64", K);
  if (K > kQ8MaxK || (long long)N * K >= (1LL << 31))
    return fail(ESM_ERR_SHAPE, "q8_pack_codes: N=%d K=%d: q exceeds 2 GB", N, K);
  if (!q || !qp) return fail(ESM_ERR_NULL, "q8_pack_codes: NULL pointer");
  if ((reinterpret_cast<uintptr_t>(q) & 7u) || !aligned16(qp))
    return fail(ESM_ERR_ALIGN, "q8_pack_codes: q must be 8-byte and qp 16-byte aligned");
  return hip_status(esm::launch_q8_pack_codes(q, qp, N, K, (hipStream_t)stream), "q8_pack_codes launch");
}

size_t q8_linear_workspace_bytes(int M, int K, int N) {
  if (M <= 0 || K <= 0 || N <= 0 || K % 64 != 0 || N % 64 != 0 || K > kQ8MaxK) return 0;
  // enough for the plain and the SwiGLU plan of the shape (their tile widths may differ)
  const Q8Plan pl = q8_plan(M, K, N), ps = q8_plan(M, K, N, true);
  const size_t a = pl.splits > 1 ? pl.bytes : 0, b = ps.splits > 1 ? ps.bytes : 0;
  return a > b ? a : b;
}

int q8_set_tile_rows(int rows) {
  if (rows != 0 && rows != 32 * esm::kQ8TileNbNarrow && rows != 32 * esm::kQ8TileNbWide)
    return fail(ESM_ERR_SHAPE, "q8_set_tile_rows: rows=%d (0, %d or %d)", rows, 32 * esm::kQ8TileNbNarrow,
                32 * esm::kQ8TileNbWide);
  g_q8_tile_rows.store(rows);
  return ok();
}

int q8_tile_rows(int M, int K, int N) {
  if (M <= 0 || K <= 0 || N <= 0) return 0;
  return 32 * q8_plan(M, K, N).nb;
}

int q8_quantize(const float* w, uint8_t* q, esm_half* s, esm_half* b, int N, int K, int group, void* stream) {
  if (N < 0 || K < 0) return fail(ESM_ERR_SHAPE, "q8_quantize: N=%d K=%d must be >= 0", N, K);
  if (group != 64) return fail(ESM_ERR_UNSUPPORTED, "q8_quantize: group=%d (supported: 64)", group);
  if (N == 0 || K == 0) return ok();
  if (K % 64 != 0) return fail(ESM_ERR_SHAPE, "q8_quantize: K=%d must be a multiple of 64", K);
  if (!w || !q || !s || !b) return fail(ESM_ERR_NULL, "q8_quantize: NULL pointer");
  if (!aligned16(w) || (reinterpret_cast<uintptr_t>(q) & 3u) || (reinterpret_cast<uintptr_t>(s) & 1u) ||
      (reinterpret_cast<uintptr_t>(b) & 1u))
    return fail(ESM_ERR_ALIGN, "q8_quantize: w must be 16-byte, q 4-byte, s and b 2-byte aligned");
  return hip_status(esm::launch_q8_quantize(w, q, H(s), H(b), N, K, (hipStream_t)stream), "q8_quantize launch");
}

int q8_dequant(const uint8_t* q, const esm_half* s, const esm_half* b, esm_half* w, int N, int K, int group,
               void* stream) {
  if (N < 0 || K < 0) return fail(ESM_ERR_SHAPE, "q8_dequant: N=%d K=%d must be >= 0", N, K);
  if (group != 64) return fail(ESM_ERR_UNSUPPORTED, "q8_dequant: group=%d (supported: 64)", group);
  if (N == 0 || K == 0) return ok();
  if (K % 64 != 0) return fail(ESM_ERR_SHAPE, "q8_dequant: K=%d must be a multiple of 64", K);
  if (!q || !s || !b || !w) return fail(ESM_ERR_NULL, "q8_dequant: NULL pointer");
  if (!aligned16(q) || !aligned16(w)) return fail(ESM_ERR_ALIGN, "q8_dequant: q, w must be 16-byte aligned");
  return hip_status(esm::launch_q8_dequant(q, H(s), H(b), H(w), N, K, (hipStream_t)stream), "q8_dequant launch");
}

int esm_timing_begin(int max_launches) {
  if (max_launches < 0 || max_launches > (1 << 20))
    return fail(ESM_ERR_SHAPE, "esm_timing_begin: max_launches=%d out of range", max_launches);
  TimingSession& t = g_timing;
  while ((int)t.events.size() < 2 * max_launches) {
    hipEvent_t e;
    const hipError_t err = hipEventCreate(&e);
    if (err != hipSuccess) return hip_status(err, "esm_timing_begin: hipEventCreate");
    t.events.push_back(e);
  }
  t.names.assign(max_launches, std::string());
  t.used = 0;
  t.cap = max_launches;
  t.armed = true;
  return ok();
}

int esm_timing_end(float* us, int cap, int* n) {
  TimingSession& t = g_timing;
  t.armed = false;
  if (!n) return fail(ESM_ERR_NULL, "esm_timing_end: NULL n");
  *n = 0;
  const int m = t.used < cap ? t.used : cap;
  if (m > 0 && !us) return fail(ESM_ERR_NULL, "esm_timing_end: NULL us");
  for (int i = 0; i < m; ++i) {
    hipError_t err = hipEventSynchronize(t.events[2 * i + 1]);
    float ms = 0.f;
    if (err == hipSuccess) err = hipEventElapsedTime(&ms, t.events[2 * i], t.events[2 * i + 1]);
    if (err != hipSuccess) return hip_status(err, "esm_timing_end: event");
    us[i] = ms * 1000.f;
  }
  *n = m;
  return ok();
}

const char* esm_timing_name(int i) {
  const TimingSession& t = g_timing;
  return (i >= 0 && i < t.used) ? t.names[i].c_str() : "";
}

}  // extern "C"
