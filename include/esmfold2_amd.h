/*
 * esmfold2_amd.h -- C ABI of the MI355X (gfx950) triangle multiplicative update
 * and 8-bit weight-only linear.
 *
 * One shared library, libesmfold2_amd.so, exports every function below. All
 * pointers are device pointers owned by the caller (the library never allocates
 * on these paths); every launch goes on the caller's HIP stream; every function
 * validates shapes, alignment and pointers before launching anything.
 *
 * Return codes: 0 = success; a negative ESM_ERR_* value = the arguments were
 * rejected before launch (nothing ran); a positive value = a hipError_t reported
 * by the runtime. esm_last_error() gives a message for the calling thread.
 * Every LayerNorm eps argument must be >= 0 (a negative or NaN eps is
 * ESM_ERR_SHAPE).
 *
 * Element types: fp16 values are IEEE binary16 (passed as uint16_t bit patterns,
 * esm_half); fp32 values are float; 8-bit codes are uint8_t.
 *
 * The interfaces these entry points replace (paths relative to the reference
 * repository, abhi0raj/esmfold2-mlx) are cited per function. The reference's
 * kernel-level interface is mx.fast.metal_kernel objects whose outputs MLX
 * allocates; here the caller allocates outputs and passes them in.
 */
#ifndef ESMFOLD2_AMD_H
#define ESMFOLD2_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint16_t esm_half;

#define ESM_OK 0
#define ESM_ERR_NULL (-1)        /* a required pointer is NULL                       */
#define ESM_ERR_SHAPE (-2)       /* a size is out of range or inconsistent           */
#define ESM_ERR_ALIGN (-3)       /* a pointer or leading dimension is misaligned     */
#define ESM_ERR_UNSUPPORTED (-4) /* a valid but not implemented configuration        */
#define ESM_ERR_DEVICE (-5)      /* no usable gfx950 device                          */

/* Message for the last non-zero return on this thread ("" if none). */
const char* esm_last_error(void);

/* Library version string and the device architecture it was built for. */
const char* esm_version(void);

/* sha256 (hex) over the sources and headers the library was compiled from; a loader
 * compares it with the current sources to refuse or rebuild a stale library. */
const char* esm_source_hash(void);

/* Bytes of caller-provided workspace tmu_forward needs for B x L x L cells with
 * c latent channels: the two operands and the contraction output [B, c, L, ld], fp16,
 * with ld = tmu_leading_dim(L), each plane sized for the larger of that layout and the
 * MFMA-fragment layout the operands take inside tmu_forward (per channel
 * ceil(L/32) x ceil(L/16) tiles of 512 halfs); for c != 128 (the wide path) a fourth
 * plane holds LN_in(z). Each plane starts 256-byte aligned. */
size_t tmu_workspace_bytes(int B, int L, int c);

/* Padded row length (elements) of the channel-major operands: L rounded up to 8,
 * so every row starts 16-byte aligned. */
int tmu_leading_dim(int L);

/*
 * Kernel (a): input LayerNorm -> C->4c projection -> sigmoid gates -> mask ->
 * channel-major operands, in one pass over z.
 *
 * Replaces, in the reference:
 *   mx.fast.layer_norm(z, ln_in_w, ln_in_b, EPS)   mlx_trunk_kernels.py:233 (mlx_trunk.py:81)
 *   proj = n @ w_in                                 mlx_trunk_kernels.py:214
 *   gate_cf(proj, mask, c) -> a, b [B, c, L, L]     mlx_trunk_kernels.py:85-97 (MSL :48-80)
 *   fast_trunk._trimul_forward lines 22-26          fast_trunk.py:22-26
 *
 * z       [B, L, L, C] fp16, cell-major (the pair tensor).
 * mask    [B, L, L] fp16 pair mask (visibility) or NULL for all ones.
 * ln_w/b  [C] fp32 norm_start weight and bias; ln_eps its eps.
 * w       [4c, C] fp16 proj_bundle.weight, rows [s_a | s_b | g_a | g_b], no bias.
 * a_out,
 * b_out   [B, c, L, ld] fp16: a = s_a*sigmoid(g_a)*m, b = s_b*sigmoid(g_b)*m.
 *         incoming = 0: the value of cell (i, k) is stored at row i, column k.
 *         incoming = 1: stored spatially transposed (row k, column i), so the
 *         contraction is the same A.B^T for both directions.
 *         Columns [L, ld) are written with zeros.
 * Supported: C = c = 128. ld % 8 == 0, ld >= L. All pointers 16-byte aligned.
 */
int tmu_project(const esm_half* z, const esm_half* mask, const float* ln_w, const float* ln_b, float ln_eps,
                const esm_half* w, esm_half* a_out, esm_half* b_out, int B, int L, int C, int c, int ld,
                int incoming, void* stream);

/*
 * Kernel (b): the triangle contraction as an fp16 MFMA batched GEMM with fp32
 * accumulation:  x[n, i, j] = scale * sum_k a[n, i, k] * b[n, j, k]
 * for n in [0, batch) (batch = B*c channels), i, j in [0, L), k in [0, ld).
 *
 * Replaces, in the reference:
 *   a @ b.swapaxes(2, 3)  (outgoing)                mlx_trunk_kernels.py:219, mlx_trunk.py:86-88
 *   a.swapaxes(2, 3) @ b  (incoming; here its operands come pre-transposed from tmu_project)
 *   self._triangular_contract(left, right)          fast_trunk.py:27-30
 *
 * a, b  [batch, L, ld] fp16, zero in columns [L, ld).
 * x     [batch, L, ldx] fp16; columns [L, ldx) are written with zeros.
 * scale fp32 factor applied to the fp32 accumulator before the one rounding to
 *       fp16 (the fp16 scheme uses 1/256, mlx_trunk.py:14-19, :47-48).
 * ld % 8 == 0, ld >= L; ldx % 8 == 0, L <= ldx <= roundup(L, 64). Pointers 16-byte aligned.
 */
int tmu_contract(const esm_half* a, const esm_half* b, esm_half* x, int batch, int L, int ld, int ldx, float scale,
                 void* stream);

/*
 * Kernels (a) and (b) with the operands in the MFMA-fragment layout tmu_forward uses
 * internally at C = c = 128 (the same launches, exposed so that a caller can run or
 * time them one at a time; the results are bit-identical to tmu_project + tmu_contract).
 * The layout, per channel plane: ceil(L/32) x ceil(L/16) tiles of 64 lanes x 8 fp16,
 * tile (rb, kb) lane l holding operand row 32 rb + l % 32, k = 16 kb + 8 (l / 32) .. +7
 * (tmu_frag_plane_elems(L) elements; rows at or past L are left unwritten and never read,
 * k at or past L is zero). Same reference interfaces as tmu_project and tmu_contract.
 *
 * tmu_project_frag: z, mask, LN and weights as tmu_project; a_out, b_out [B * c] planes.
 * tmu_contract_frag: a, b [batch] planes; x [batch, L, ldx] as tmu_contract, columns
 *   [L, ldx) written with zeros; ldx % 8 == 0, L <= ldx <= roundup(L, 32).
 * Supported: C = c = 128 (project). Pointers 16-byte aligned.
 */
size_t tmu_frag_plane_elems(int L);
int tmu_project_frag(const esm_half* z, const esm_half* mask, const float* ln_w, const float* ln_b, float ln_eps,
                     const esm_half* w, esm_half* a_out, esm_half* b_out, int B, int L, int C, int c,
                     int incoming, void* stream);
int tmu_contract_frag(const esm_half* a, const esm_half* b, esm_half* x, int batch, int L, int ldx, float scale,
                      void* stream);

/*
 * Kernel (c): norm_mix LayerNorm over c of the channel-major contraction ->
 * proj_emit -> * sigmoid(proj_gate(LN_in(z))) [-> * mask] [-> + z], written
 * cell-major.
 *
 * Replaces, in the reference:
 *   ln_cf_to_cl(contracted, ln_mix_w, ln_mix_b, mix_eps)   mlx_trunk_kernels.py:152-160 (MSL :107-147)
 *   mixed @ w_emit; n @ w_out_gate                         mlx_trunk_kernels.py:224-225
 *   resgate_ln's z + m*sigmoid(g)  (residual = 1)          mlx_trunk_kernels.py:165-190
 *   fast_trunk._trimul_forward lines 31-32                 fast_trunk.py:31-32
 *
 * x        [B, c, L, ldx] fp16 contraction output (as written by tmu_contract).
 * z        [B, L, L, C] fp16 pair tensor (the gate is recomputed from LN_in(z)).
 * mask     [B, L, L] fp16 or NULL; used only when out_mask != 0 (the reference
 *          does not mask the update: off by default).
 * ln_in_*  norm_start (C); ln_mix_* norm_mix (c); eps values as given.
 * w_emit   [C, c] fp16 proj_emit.weight; w_gate [C, C] fp16 proj_gate.weight.
 * out      [B, L, L, C] fp16: the update, or z + update when residual != 0
 *          (out may alias z only when residual != 0).
 * Supported: C = c = 128.
 */
int tmu_epilogue(const esm_half* x, int ldx, const esm_half* z, const esm_half* mask, const float* ln_in_w,
                 const float* ln_in_b, float ln_in_eps, const float* ln_mix_w, const float* ln_mix_b,
                 float ln_mix_eps, const esm_half* w_emit, const esm_half* w_gate, esm_half* out, int B, int L,
                 int C, int c, int residual, int out_mask, void* stream);

/*
 * One whole triangle multiplicative update: kernels (a), (b), (c) in sequence on
 * `stream`, with the fp16 range scheme of the reference's fp16 trunk (the
 * contraction is stored as x/256 and norm_mix's eps divided by 256^2, an exact
 * identity: mlx_trunk.py:14-19, :47-48, :114).
 *
 * Replaces fast_trunk._trimul_forward (fast_trunk.py:19-32), i.e. the per-module
 * forward(pair_grid, visibility) -> update the reference's variant mechanism
 * binds (fast_trunk.py:57), and mlx_trunk_kernels._trimul (mlx_trunk_kernels.py:210-229).
 *
 * workspace: tmu_workspace_bytes(B, L, c) bytes, 256-byte aligned, caller-owned.
 * outgoing: 1 = "outgoing edges" update, 0 = "incoming edges".
 * Supported: C = c = 128 (kernels (a), (b), (c)), or C = c a multiple of 128 up to 512
 * (ESMFold2's trunk is 256 wide, mlx_trunk.py:3-5): the wide path, five launches with
 * the same arithmetic (LN_in(z) -> gated projection stored channel-major -> kernel (b)
 * -> LN_mix over channels turned cell-major -> emit and gate GEMMs with the residual).
 * L <= 4096 and B * c <= 65535; B * L * L * C is bounded only by memory (each kernel
 * addresses its tile or channel plane from a 64-bit base).
 */
int tmu_forward(const esm_half* z, const esm_half* mask, const float* ln_in_w, const float* ln_in_b, float ln_in_eps,
                const esm_half* w_bundle, const float* ln_mix_w, const float* ln_mix_b, float ln_mix_eps,
                const esm_half* w_emit, const esm_half* w_gate, esm_half* out, void* workspace, int B, int L, int C,
                int c, int outgoing, int residual, int out_mask, void* stream);

/*
 * The two triangle updates of a trunk block, out = z1 + T_in(z1), z1 = z + T_out(z):
 * tmu_forward for the outgoing update (residual, into out), then for the incoming one (in
 * place on out), in one call.
 *
 * Replaces, in the reference:
 *   block_forward's first two lines                 mlx_trunk.py:94-95
 *   fast_trunk's patched tri_mul_out, tri_mul_in    fast_trunk.py:19-32, :57 (called
 *                                                   with the residual by the trunk block)
 *
 * o_* are the outgoing update's parameters and i_* the incoming update's, each as
 * tmu_forward takes them (o_out_mask / i_out_mask as its out_mask). out may be z itself.
 * workspace: tmu_workspace_bytes(B, L, c) bytes, 256-byte aligned. Shape limits as
 * tmu_forward; every argument is checked before the first launch.
 */
int tmu_pair_forward(const esm_half* z, const esm_half* mask, const float* o_ln_in_w, const float* o_ln_in_b,
                     float o_ln_in_eps, const esm_half* o_w_bundle, const float* o_ln_mix_w, const float* o_ln_mix_b,
                     float o_ln_mix_eps, const esm_half* o_w_emit, const esm_half* o_w_gate, int o_out_mask,
                     const float* i_ln_in_w, const float* i_ln_in_b, float i_ln_in_eps, const esm_half* i_w_bundle,
                     const float* i_ln_mix_w, const float* i_ln_mix_b, float i_ln_mix_eps, const esm_half* i_w_emit,
                     const esm_half* i_w_gate, int i_out_mask, esm_half* out, void* workspace, int B, int L, int C,
                     int c, void* stream);

/*
 * tmu_forward and tmu_pair_forward with the workspace's size: a workspace_bytes below
 * tmu_workspace_bytes(B, L, c) returns ESM_ERR_SHAPE before any launch. The size depends on
 * the width (the C >= 256 path keeps a fourth plane) and on the operand layout, so a caller
 * that keeps its own buffer across shapes or library versions should use these forms.
 * Same reference call sites as the unsized forms above.
 */
int tmu_forward_ws(const esm_half* z, const esm_half* mask, const float* ln_in_w, const float* ln_in_b,
                   float ln_in_eps, const esm_half* w_bundle, const float* ln_mix_w, const float* ln_mix_b,
                   float ln_mix_eps, const esm_half* w_emit, const esm_half* w_gate, esm_half* out, void* workspace,
                   size_t workspace_bytes, int B, int L, int C, int c, int outgoing, int residual, int out_mask,
                   void* stream);
int tmu_pair_forward_ws(const esm_half* z, const esm_half* mask, const float* o_ln_in_w, const float* o_ln_in_b,
                        float o_ln_in_eps, const esm_half* o_w_bundle, const float* o_ln_mix_w,
                        const float* o_ln_mix_b, float o_ln_mix_eps, const esm_half* o_w_emit,
                        const esm_half* o_w_gate, int o_out_mask, const float* i_ln_in_w, const float* i_ln_in_b,
                        float i_ln_in_eps, const esm_half* i_w_bundle, const float* i_ln_mix_w,
                        const float* i_ln_mix_b, float i_ln_mix_eps, const esm_half* i_w_emit,
                        const esm_half* i_w_gate, int i_out_mask, esm_half* out, void* workspace,
                        size_t workspace_bytes, int B, int L, int C, int c, void* stream);

/*
 * Kernel (e): the pair transition, out = z + W3 act(W1 LN(z)) on every cell, with
 * act = ReLU (w2 == NULL: transformers' EsmFoldResidueMLP without biases, the
 * block-stack workload's 128 -> H -> 128 MLP) or SwiGLU, act = silu(W1 h) * (W2 h)
 * (the reference's transition: fast_trunk.py:35-42 with w1 = ffn.w12.weight[:H],
 * w2 = ffn.w12.weight[H:], w3 = ffn.w3.weight; mlx_trunk.py:96-99 and its addmm
 * residual, mlx_trunk_kernels.py:236-239). No biases (fast_trunk.py:59).
 *
 * z, out [B, L, L, C] fp16 cell-major (out may be z); ln_w, ln_b [C] fp32;
 * w1, w2 [H, C] fp16; w3 [C, H] fp16 (torch [out, in] layouts). fp32 statistics and
 * accumulation; the hidden activations and the output are each rounded once to fp16.
 * Without a workspace: C = 128 with ReLU at H = 256 or 512, or SwiGLU at H = 256 (one
 * register-resident kernel). Other shapes need pair_transition_ws.
 */
int pair_transition(const esm_half* z, esm_half* out, const float* ln_w, const float* ln_b, float eps,
                    const esm_half* w1, const esm_half* w2, const esm_half* w3, int B, int L, int C, int H,
                    void* stream);

/*
 * pair_transition for every supported shape: C a multiple of 128 up to 512 and H a
 * multiple of 32 (ESMFold2's 256-wide trunk with its SwiGLU hidden width). The shapes
 * pair_transition covers run its kernel and ignore the workspace; the others run LN(z),
 * then one GEMM with the activation fused (hidden [cells, H] fp16, rounded once), then one
 * with the residual fused, in `workspace` of at least
 * pair_transition_workspace_bytes(B, L, C, H, swiglu) bytes (256-byte aligned; 0 bytes
 * when none is needed). out may be z.
 */
size_t pair_transition_workspace_bytes(int B, int L, int C, int H, int swiglu);
int pair_transition_ws(const esm_half* z, esm_half* out, const float* ln_w, const float* ln_b, float eps,
                       const esm_half* w1, const esm_half* w2, const esm_half* w3, int B, int L, int C, int H,
                       void* workspace, size_t workspace_bytes, void* stream);

/*
 * Kernel (d): MLX-affine 8-bit weight-only linear, y = x . W^T with
 * W[n, k] = RN_fp16(s[n, k/64] * q[n, k] + b[n, k/64]) (dequantised in registers,
 * one fp16 FMA rounding) and fp32 accumulation; y rounded once to fp16.
 *
 * Replaces mx.quantized_matmul(x, w, s, b, transpose=True, group_size=64, bits=8)
 * (mlx_esmc.py:78-81; weights from mlx_esmc.py:53-75). The reference packs codes
 * four per uint32, little-endian: byte-identical to the row-major uint8 [N, K]
 * taken here.
 *
 * x [M, K] fp16; q [N, K] uint8; s, b [N, K/group] fp16; y [M, N] fp16.
 * Supported: group = 64, K % 64 == 0, N % 64 == 0, M >= 1.
 */
int q8_linear(const esm_half* x, const uint8_t* q, const esm_half* s, const esm_half* b, esm_half* y, int M, int K,
              int N, int group, void* stream);

/*
 * q8_linear with the two optional speed-ups a long-lived caller (a layer holding its
 * weights) can afford:
 *   sb: the scales and biases pre-packed by q8_pack_scales (once per weight matrix);
 *       NULL reads them from s and b (slower: 128-160 scattered rows per 128-wide step).
 *   workspace: for shapes whose output tiles (64 x 128 or 64 x 160, q8_tile_rows) are too
 *       few to fill the GPU (e.g. M = 238, N = 2560), K is split over several workgroups whose fp32
 *       partials go through the workspace and are summed in split order by a second
 *       kernel on the same stream (deterministic). q8_linear_workspace_bytes(M, K, N)
 *       bytes, 256-byte aligned, no initialisation needed; NULL runs unsplit. Calls
 *       that share a workspace must not overlap in time.
 * s and b are required either way. Same semantics and result as q8_linear
 * (mx.quantized_matmul, mlx_esmc.py:78-81); packed or not, the bits are identical.
 */
int q8_linear_ws(const esm_half* x, const uint8_t* q, const esm_half* s, const esm_half* b, const uint32_t* sb,
                 esm_half* y, int M, int K, int N, int group, void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes q8_linear_ws (or q8_linear_swiglu_packed_ws) uses for this shape on the
 * current device (0: none). */
size_t q8_linear_workspace_bytes(int M, int K, int N);

/*
 * The weight rows per output tile the launch plan picks for this shape on the current
 * device, 128 or 160: the width with the lower estimated time, rounds of the GPU's CUs x
 * 128-wide K steps per workgroup x a step's time (a 128-row step ~0.9 of a 160-row one),
 * plus, where K is split, the fp32 partials' write and read (160 always for the SwiGLU-pair
 * call). At M = 238: 128 for N = 7680 and for N = 2560 at K = 2560, 160 for N = 10240 and for
 * N = 2560 at K = 5120 or 10240.
 * Either width gives the same bits when K is not split (it only changes which workgroup
 * computes an output); with a K split the split count, and so the fp32 summation order,
 * can differ. q8_set_tile_rows(128 or 160) fixes the width for every later plan of this
 * process (0 restores the choice; tests and tuning). No reference counterpart: the
 * reference's quantized_matmul (mlx_esmc.py:78-81) tiles inside MLX.
 */
int q8_tile_rows(int M, int K, int N);
int q8_set_tile_rows(int rows);

/*
 * The GEMM of q8_linear_ws without its last step: the fp32 partial sums of y go to
 * parts [*splits, M, N] (split s covers a contiguous range of K's groups; *splits is the
 * split count this device's plan uses, 1 when the tiles already fill the GPU) and are
 * not summed. esmc_layer_norm_parts consumes them, summing in split order and rounding
 * once to fp16, which gives the bits q8_linear_ws writes to y. Together the two replace,
 * in the reference, a block's `wo(o)` / `w2(...)` (mx.quantized_matmul, mlx_esmc.py:78-81)
 * followed by its residual add and LayerNorm (:97-98, :102 and the next block's :91),
 * without the separate reduction kernel and the fp16 y in between.
 * parts: q8_linear_partials_bytes(M, K, N) bytes, 256-byte aligned, no initialisation
 * needed; sb as in q8_linear_ws (NULL allowed).
 */
size_t q8_linear_partials_bytes(int M, int K, int N);
int q8_linear_partials(const esm_half* x, const uint8_t* q, const esm_half* s, const esm_half* b, const uint32_t* sb,
                       float* parts, size_t parts_bytes, int* splits, int M, int K, int N, int group, void* stream);

/*
 * Packs s and b [N, K/group] fp16 into sb [ceil(N/32), K/group, 32] uint32 words
 * (b << 16 | s; rows past N are 0): per 32-row block, so a tile of either width reads a
 * step's words as 256-byte contiguous pieces. A layout cache of the reference's fp16
 * scales/biases (mlx_esmc.py:53-75), built once per weight matrix. group = 64.
 */
size_t q8_packed_scales_bytes(int N, int K);
int q8_pack_scales(const esm_half* s, const esm_half* b, uint32_t* sb, int N, int K, int group, void* stream);

/*
 * Packs the codes q [N, K] (MLX's layout, one byte per weight) into qp in the order the
 * GEMM's matrix-core fragments take them: per 32-row block and step of two groups (128 k),
 * 4 chunks of 1 KB (one per wave), one 16-byte piece per lane; rows past N and groups past
 * K/group are 0. Independent of the tile width. q8_packed_codes_bytes(N, K) bytes (about N K; 0 for an unsupported shape), qp
 * 16-byte aligned, q 8-byte aligned. A layout cache of the reference's 8-bit weights
 * (mlx_esmc.py:53-75), built once per weight matrix like q8_pack_scales. group = 64.
 */
size_t q8_packed_codes_bytes(int N, int K);
int q8_pack_codes(const uint8_t* q, uint8_t* qp, int N, int K, int group, void* stream);

/*
 * q8_linear_ws and q8_linear_partials on packed weights: qp from q8_pack_codes and sb from
 * q8_pack_scales of the same matrix (both required; q, s and b are not read). Each wave
 * loads its matrix-core fragments of the codes straight into registers, so only x and the
 * scales pass through LDS. Same plan, workspace, partials and results, bit for bit, as the
 * [N, K] forms; the same reference calls (mlx_esmc.py:78-81).
 */
int q8_linear_packed_ws(const esm_half* x, const uint8_t* qp, const uint32_t* sb, esm_half* y, int M, int K, int N,
                        int group, void* workspace, size_t workspace_bytes, void* stream);
int q8_linear_packed_partials(const esm_half* x, const uint8_t* qp, const uint32_t* sb, float* parts,
                              size_t parts_bytes, int* splits, int M, int K, int N, int group, void* stream);

/*
 * The block's first FFN linear and its SwiGLU in one call: y [M, N/2] = silu(x W_gate^T) *
 * (x W_up^T), W = [gate; up] rows [N, K] (mlx_esmc.py:100-101, the `w1` linear then
 * silu(x1) * x2). qp and sb are q8_pack_codes / q8_pack_scales of the rows in SwiGLU pair
 * order: each 160-row tile holds gate rows 80 t .. 80 t + 79, then up rows 80 t .. 80 t + 79
 * (N a multiple of 160). Same bits as q8_linear_ws on the [gate; up] rows followed by
 * esmc_swiglu: the gate and up sums round to fp16 before the gating, unsplit in the GEMM's
 * epilogue, split-K in the reduction of the partials (workspace as for q8_linear_ws at M, K, N).
 */
int q8_linear_swiglu_packed_ws(const esm_half* x, const uint8_t* qp, const uint32_t* sb, esm_half* y, int M, int K,
                               int N, int group, void* workspace, size_t workspace_bytes, void* stream);

/*
 * The ESMC transformer block's other kernels (mlx_esmc.py:84-102), around q8_linear.
 *
 * esmc_layer_norm: with y, x_out = x + alpha * y (fp32 residual, y fp16: the scaled
 *   residual adds `x + (wo(o) / res_scale)`, mlx_esmc.py:97, :102); then
 *   h = LN(x_out or x; w, b, eps) in fp32, rounded to fp16 (mx.fast.layer_norm,
 *   :91, :98), or kept in fp32 in h_fp32 (the final norm, :195); exactly one of h,
 *   h_fp32 is given. x, x_out [M, D] fp32 (x_out may be x); y, h [M, D] fp16;
 *   w, b [D] fp32 (b may be NULL). D % 8 == 0, D <= 8192.
 * esmc_qk_rope: qkv [B*L, 3D] fp16 (the wqkv output, rows [q | k | v]); QK-LayerNorm
 *   over the full width D with weights only (:93-94), fp32 statistics; NeoX rotary
 *   embedding (mx.fast.rope traditional=False, base rope_base, positions 0..L-1,
 *   :96-97; the angle in fp32, its sine and cosine from the hardware's, on the angle in
 *   revolutions); q, k, v written head-major [B, H, L, 64] fp16. head_dim = 64, D <= 4096;
 *   qkv, q_ln, k_ln, q, k, v 16-byte aligned.
 * esmc_attention: o = softmax(q k^T * scale, mask) v per (batch, head) (:98,
 *   mx.fast.scaled_dot_product_attention), with token i attending to j iff
 *   sequence_id[b, i] == sequence_id[b, j] (:186-191; NULL = no mask); fp32 scores and
 *   softmax, probabilities rounded to fp16 for the second product; o [B, L, H*64] fp16.
 *   head_dim = 64, L <= 65536 (keys in passes of 512 with an online softmax beyond 512).
 * esmc_swiglu: y = silu(x1) * x2 with x12 = [x1 | x2] rows [M, 2F] fp16 (:100-101), in
 *   fp32, one rounding; y [M, F]. F % 8 == 0.
 */
int esmc_layer_norm(const float* x, const esm_half* y, float alpha, float* x_out, const float* w, const float* b,
                    float eps, esm_half* h, float* h_fp32, int M, int D, void* stream);
/*
 * esmc_layer_norm with y given as q8_linear_partials' output: y = fp16(sum over s of
 * y_parts[s]) in split order, then x_out = x + alpha * y and h = LN(x_out) exactly as
 * above (the same bits as q8_linear_ws followed by esmc_layer_norm). y_parts
 * [splits, M, D] fp32, 16-byte aligned; splits >= 1; x_out required.
 */
int esmc_layer_norm_parts(const float* x, const float* y_parts, int splits, float alpha, float* x_out, const float* w,
                          const float* b, float eps, esm_half* h, float* h_fp32, int M, int D, void* stream);
int esmc_qk_rope(const esm_half* qkv, const float* q_ln, const float* k_ln, float eps, esm_half* q, esm_half* k,
                 esm_half* v, int B, int L, int n_heads, int head_dim, float rope_base, void* stream);
int esmc_attention(const esm_half* q, const esm_half* k, const esm_half* v, const int* sequence_id, esm_half* o, int B,
                   int L, int n_heads, int head_dim, float scale, void* stream);
int esmc_swiglu(const esm_half* x12, esm_half* y, int M, int F, void* stream);

/*
 * The recycling step around the trunk.
 *
 * parcae_step: z_out = a * z + LN(z_init + refined; ln_w, ln_b, eps) @ B^T on every
 *   cell (var_6b_mlx_loop.py:67-71: u = z_init + lm_encoder(lm_z), the "parcae"
 *   linear recurrence, fp32). z, z_init, refined, z_out [B, L, L, C] fp32 (z_out may be
 *   z); ln_w, ln_b, a [C] fp32; b_mat [C, C] fp16 (torch [out, in]). LayerNorm in fp32,
 *   its output and B rounded to fp16 for the MFMA, fp32 accumulation and update. C = 128 or 256.
 * distogram_expected_distance: ed = softmax((r + r^T) @ W^T + bias) . centers per pair
 *   (var_6b_mlx_loop.py:74-76; var_adaptive_loops.py:41-46), r^T swapping the two
 *   residue axes. r [B, L, L, C] fp32 (the readout or the coda output); w [nbins, C] fp16
 *   (the head's weight); bias, centers [nbins] fp32; ed [B, L, L] fp32. The pair sums are
 *   rounded to fp16 for the MFMA; logits and softmax in fp32. C = 128 or 256, nbins 64 or 128.
 *   ed is exactly symmetric: each pair j >= i is computed once and stored to ed[i,j] and
 *   ed[j,i] (r[i,j] + r[j,i] is the same fp32 sum either way round), so r is read once.
 * abs_diff_quantile: out[0] = the q-th quantile of |x - y| (y NULL: of |x|) over n values,
 *   linear interpolation between the two nearest order statistics, as torch.quantile
 *   (the exit signal: var_6b_mlx_loop.py:79-85 with q = 0.95, var_adaptive_loops.py:116).
 *   Exact (order statistics by radix selection). x, y [n] fp32; out one fp32. A NaN difference
 *   orders above +inf, as the sort of the MLX loop's p95 (var_6b_mlx_loop.py:78-84) orders it
 *   (torch.quantile would return NaN instead).
 */
int parcae_step(const float* z, const float* z_init, const float* refined, const float* ln_w, const float* ln_b,
                float eps, const float* a, const esm_half* b_mat, float* z_out, int B, int L, int C, void* stream);
int distogram_expected_distance(const float* r, const esm_half* w, const float* bias, const float* centers, float* ed,
                                int B, int L, int C, int nbins, void* stream);
int abs_diff_quantile(const float* x, const float* y, size_t n, float q, float* out, void* stream);

/*
 * q8_linear_ws without a workspace, for callers that cannot allocate device memory (code
 * under HIP graph capture, serving loops that forbid allocation). No counterpart in the
 * reference: its MLX quantized_matmul allocates its own outputs. Same plan and same bits
 * as q8_linear_ws with a workspace; the split-K partials live in a static device array of
 * ESM_Q8_NOALLOC_SCRATCH_BYTES per GPU (taken by the library for the life of the
 * process). A shape whose partials exceed it is refused with ESM_ERR_SHAPE (with 256
 * compute units the plan needs at most about 10.5 MB). Nothing is allocated and nothing
 * needs clearing between calls; calls that overlap in time on one GPU share the array and
 * race, so a caller serialises them (one stream, or its own ordering).
 */
#define ESM_Q8_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)
int q8_linear_noalloc(const esm_half* x, const uint8_t* q, const esm_half* s, const esm_half* b, const uint32_t* sb,
                      esm_half* y, int M, int K, int N, int group, void* stream);

/*
 * Quantise fp32 weights to the 8-bit layout q8_linear reads: MLX's affine scheme, group
 * 64 along K, scales and biases rounded to fp16.
 *
 * Replaces, in the reference:
 *   wq, scales, biases = mx.quantize(W, group_size=64, bits=8)   mlx_esmc.py:73
 *   scales.astype(mx.float16), biases.astype(mx.float16)         mlx_esmc.py:74
 *
 * Per group of 64 (fp32 arithmetic, IEEE division, rint = round half to even):
 *   scale = max((max - min) / 255, 1e-7), negated unless |min| > |max|;
 *   edge = min if |min| > |max| else max;  q0 = rint(edge / scale);
 *   q0 != 0: scale = edge / q0, bias = edge;  q0 == 0: bias = 0;
 *   q = clamp(rint((w - bias) / scale), 0, 255).
 * w [N, K] fp32 (torch's [out, in] layout), 16-byte aligned; q [N, K] uint8 (4-byte
 * aligned); s, b [N, K/64] fp16. group = 64, K % 64 == 0.
 */
int q8_quantize(const float* w, uint8_t* q, esm_half* s, esm_half* b, int N, int K, int group, void* stream);

/*
 * Dequantise only: w[n, k] = RN_fp16(s[n, k/group] * q[n, k] + b[n, k/group]),
 * the exact weights q8_linear multiplies by (for the bit-exact check).
 * q [N, K] uint8; s, b [N, K/group] fp16; w [N, K] fp16. group = 64, K % 64 == 0.
 */
int q8_dequant(const uint8_t* q, const esm_half* s, const esm_half* b, esm_half* w, int N, int K, int group,
               void* stream);

/*
 * Kernel timing for measurement (no counterpart in the reference, whose timings are wall
 * clocks around whole folds, tools/bench_e2e.py:120-127). esm_timing_begin(n) arms the calling
 * thread: its next n kernel launches through this library carry start/stop events that the
 * runtime stamps with the kernel's own begin and end (hipExtLaunchKernelGGL), i.e. the
 * durations a profiler's kernel trace reports. esm_timing_end waits for them and writes up to
 * `cap` durations in microseconds, in launch order, and their count to *n; it disarms the
 * thread. esm_timing_name(i) is the i-th timed launch's kernel name. Not for use under HIP
 * graph capture. Events are created by the first begin and reused.
 */
int esm_timing_begin(int max_launches);
int esm_timing_end(float* us, int cap, int* n);
const char* esm_timing_name(int i);

#ifdef __cplusplus
}
#endif

#endif /* ESMFOLD2_AMD_H */
