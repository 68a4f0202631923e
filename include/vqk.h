/* vqk.h -- C ABI of the MI355X (gfx950) VQ weight-decode library, libvqk.so.
 *
 * Plain pointers and sizes only. Device pointers are HIP device memory;
 * `stream` is a hipStream_t passed as void* (NULL = the default stream).
 * Every entry point validates its arguments on the host and returns a status
 * before anything is launched; no entry point allocates device memory --
 * callers that need scratch pass a workspace sized by the matching
 * *_workspace query (the one exception, vqk_moe_decode_layer_noalloc, uses
 * a library-owned device array instead). Kernels are re-entrant.
 *
 * Each entry point cites the reference interface it replaces (paths are
 * relative to the reference checkout; vq_switch.py, vq_dense.py and vq_pack.py
 * live in src/vqlab/runtime/).
 */
#ifndef VQK_H
#define VQK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes: map 1:1 onto the reference's exceptions --------------
 * VQK_ENOTIMPL  NotImplementedError: unsupported d / bits / geometry
 *               (vq_switch.py:3106-3109, 3350-3362)
 * VQK_EINVAL    ValueError: WPR / column / shape mismatch
 *               (vq_switch.py:3124-3128, 3365-3368; vq_dense.py:330-331)
 * VQK_ESHARDED  RuntimeError: codebook rows differ from the module's K
 *               (vq_switch.py:5285-5296; vq_dense.py:349-353)
 * VQK_EDEVICE   a HIP runtime call failed (launch, stream)
 * VQK_ENOSPACE  the workspace passed is smaller than *_workspace reported */
#define VQK_OK        0
#define VQK_ENOTIMPL  1
#define VQK_EINVAL    2
#define VQK_ESHARDED  3
#define VQK_EDEVICE   4
#define VQK_ENOSPACE  5

/* ---- element types ------------------------------------------------------ */
#define VQK_F16   0
#define VQK_BF16  1
#define VQK_F32   2
#define VQK_U8    3
#define VQK_U16   4
#define VQK_U32   5
#define VQK_I32   6
#define VQK_I64   7

/* Output rounding flag, OR'd into the y_type of any GEMV / GEMM / layer entry
 * point: the fp32 result is rounded to fp16 first, then into y's type -- the
 * arithmetic of the reference's default decode path, whose fused kernels
 * return fp16 that the caller then casts to x's dtype (vq_switch.py:5306-5308,
 * 5423). Without it a result is rounded once, from fp32, into y's type (the
 * reference with VQ_DECODE_BF16IO=1, vq_switch.py:4421, 5303-5306). */
#define VQK_VIA_F16 0x100

/* Wide-activation flag, OR'd into the x_type of vqk_moe_expert_gemv /
 * vqk_dense_gemv for d = 4 and d = 8 modules (VQK_EINVAL at d = 2): x enters
 * the products unrounded -- bf16 and fp32 activations widened exactly to
 * fp32, each codebook half widened to fp32, fp32 multiply-adds -- instead of
 * being narrowed to fp16 first. It is the arithmetic of the reference's
 * float-staged decode kernels -- the unpacked d4 kernel for K <= 1024
 * (_SRC_FUSED, vq_switch.py:106-150) and the d8 kernels for K > 1024
 * (153-237, 1316-1354, 1424-1660) -- which VQ_DECODE_BF16IO feeds bf16 x
 * uncast (vq_switch.py:4412-4417, 5306); its other decode kernels (d2,
 * packed or K > 1024 d4, d8 with K <= 1024) stage x as fp16 and round it
 * in-kernel, and its grouped prefill converts bf16 x to fp16 on stage-in
 * even under VQ_GEMMSEG_BF16IO (vq_switch.py:4364-4372). vqk_switch_apply
 * sets it by that rule (see vqk_options.decode_bf16io), and
 * vqk_linear_apply for d8 linears, which the reference runs through
 * decode-then-matmul in x's type. No other entry point accepts it. */
#define VQK_X_KEEP 0x200

/* One VQ-coded linear, or a stack of E expert linears sharing one codebook
 * (VQSwitchLinear, vq_switch.py:5198-5234; VQLinear, vq_dense.py:322-334).
 *
 *   codes      pack_bits == 0: VQK_U8 / VQK_U16 [E, OUT, NSUB], NSUB = IN / D
 *              pack_bits  > 0: VQK_U32 [E, OUT, WPR] words, WPR =
 *                              ceil(NSUB / 32) * pack_bits (vq_pack.py:11-27)
 *              with row_table: compact live rows [n_live, NSUB or WPR]
 *   code_cols  the codes tensor's last dimension as stored; it must equal
 *              NSUB (unpacked) or WPR (packed), else VQK_EINVAL
 *              (vq_switch.py:3124-3128)
 *   codebook   fp16 [K, D], D in {2, 4, 8}; ONE per module, shared by all
 *              experts (vq_switch.py:5-8)
 *   scales     fp16 [E, OUT, IN / group] (compact [n_live, IN / group])
 *   row_table  int32 [E, OUT]: compact row of (expert, row), -1 = dead row
 *              (skipzero, vq_switch.py:5206-5214); NULL = expanded tensors
 *   k_expect   the codebook row count the module was built with; a
 *              different K is a sharded codebook (VQK_ESHARDED). 0 = K.
 * A dense linear is E = 1. */
typedef struct vqk_weights {
    const void     *codes;
    int64_t         code_cols;
    int32_t         code_type;
    int32_t         pack_bits;
    const uint16_t *codebook;
    int64_t         K;
    int32_t         D;
    int32_t         group;
    const uint16_t *scales;
    int64_t         E;
    int64_t         OUT;
    int64_t         IN;
    const int32_t  *row_table;
    int64_t         n_live;
    int64_t         k_expect;
} vqk_weights;

/* Library identification and the calling thread's last error message. */
const char *vqk_version(void);
const char *vqk_last_error(void);

/* ---- a1: widths ----------------------------------------------------------
 * bits_for_k: vq_pack.py:34-38. words_per_row: vq_pack.py:41-45 (returns -1
 * for bad arguments). pack_bits_for: codepack.py:22-30 (0 = stays unpacked). */
int     vqk_bits_for_k(int64_t k, int32_t *bits);
int64_t vqk_words_per_row(int64_t nsub, int32_t bits);
int     vqk_pack_bits_for(int64_t k, int64_t nsub, int32_t pack_unaligned,
                          int32_t *bits);

/* ---- a2/a3: index packing (vq_pack.pack / vq_pack.unpack, vq_pack.py:48-97)
 * rows = E * OUT flattened. Codes are uint16 on input (any width 1..16);
 * unpack writes uint8 when bits <= 8 else uint16, like vq_pack.unpack.
 * *_host work on host memory, the others launch on `stream`. */
int vqk_pack_host(const uint16_t *codes, int64_t rows, int64_t nsub,
                  int32_t bits, uint32_t *packed);
int vqk_unpack_host(const uint32_t *packed, int64_t rows, int64_t nsub,
                    int32_t bits, void *codes);
int vqk_pack(const uint16_t *codes, int64_t rows, int64_t nsub, int32_t bits,
             uint32_t *packed, void *stream);
int vqk_unpack(const uint32_t *packed, int64_t rows, int64_t nsub,
               int32_t bits, void *codes, void *stream);

/* ---- a4: dequantisation, bit-exact W = fp16(f32(cb[c]) * f32(s)) ----------
 * vqk_dequant: wdec_decode (vq_switch.py:3517-3544) -- rows [r0, r0 + rows)
 *   of the flattened [E * OUT] module into out [rows, IN] fp16.
 * vqk_dequant_experts: _decode_chunk (vq_switch.py:4725-4782) -- experts
 *   eidx[0..ne) (device uint32) into out [ne, OUT, IN] fp16.
 * Dead skipzero rows decode to +0. */
int vqk_dequant(const vqk_weights *w, int64_t r0, int64_t rows,
                uint16_t *out, void *stream);
int vqk_dequant_experts(const vqk_weights *w, const uint32_t *eidx,
                        int64_t ne, uint16_t *out, void *stream);

/* ---- a10: dense fused GEMV, _dense_fused (vq_switch.py:3339-3434) ----------
 * y[N, OUT] = x[N, IN] . W^T for E == 1, fp32 accumulation; x and y types in
 * {VQK_F16, VQK_BF16, VQK_F32}. */
int vqk_dense_gemv(const vqk_weights *w, const void *x, int32_t x_type,
                   int64_t N, void *y, int32_t y_type, void *stream);

/* ---- a5-a9: routed-expert fused GEMV, _fused (vq_switch.py:2919-3249) -------
 * Pair n (n < N) multiplies token row n / xkrep of x [T, IN] with expert
 * eidx[n] (device uint32): y[n, :] = x[n / xkrep] . W_eidx[n]^T. xkrep = 1
 * is the historical contract (x already has N rows); xkrep = k is the XKREP
 * form (vq_switch.py:4422-4451). Requires N == T * xkrep. */
int vqk_moe_expert_gemv(const vqk_weights *w, const void *x, int32_t x_type,
                        int64_t T, const uint32_t *eidx, int64_t N,
                        int64_t xkrep, void *y, int32_t y_type, void *stream);

/* ---- a12: routed-expert grouped GEMM, _gemmseg_prefill (vq_switch.py:4569-4722)
 * Same contract and output order as vqk_moe_expert_gemv, for large N: the
 * pairs are count-sorted by expert ON DEVICE (no host sync, replacing the
 * host argsort at vq_switch.py:5383-5388 and the tile build at 4590-4610),
 * and each expert tile's weights are decoded bit-exactly straight into fp16
 * matrix-core operands (codebook in LDS, or its first part in LDS and the
 * rest gathered from L2), fp32 accumulation. The sort picks the tile rows on
 * device (16, or for d8 tables beyond LDS under a thin routing 4 or 8, the
 * larger where it saves decoding an expert's rows twice). The workspace is
 * 16-byte aligned. */
int vqk_grouped_gemm_workspace(const vqk_weights *w, int64_t N, size_t *bytes);
int vqk_grouped_gemm(const vqk_weights *w, const void *x, int32_t x_type,
                     int64_t T, const uint32_t *eidx, int64_t N, int64_t xkrep,
                     void *y, int32_t y_type, void *workspace, size_t ws_bytes,
                     void *stream);

/* ---- a11: dense large-N path, _decode_matmul (vq_dense.py:262-312) ---------
 * y[N, OUT] = x[N, IN] . W^T for E == 1. Up to 64 rows: W is decoded straight
 * into matrix-core operands (no workspace, x rounded to fp16 as the fused
 * kernels take it). Above (and for shapes that path refuses): the reference's
 * decode-then-matmul, `xf @ w.T.astype(xf.dtype)` -- W is dequantised into the
 * workspace panel by panel in x's arithmetic type and multiplied by libvqk's
 * matrix-core GEMM with fp32 accumulation: fp16 x against the bit-exact fp16
 * W, bf16 x against W rounded once to bf16, fp32 x through split bf16
 * operands (x to 16 significant bits, W exactly; three products per term).
 * x is staged into the workspace when it is fp32, not 16-byte aligned or IN
 * is not a multiple of 64 (rows zero-padded). vqk_dense_gemm_workspace gives a
 * size that holds the whole weight as one panel for any activation type; a
 * smaller workspace that still holds the staged x plus 128 weight rows runs
 * in more panels, less (or none) is VQK_ENOSPACE; it is 16-byte aligned. No
 * host synchronisation, no allocation, no state kept between calls. */
int vqk_dense_gemm_workspace(const vqk_weights *w, int64_t N, size_t *bytes);
int vqk_dense_gemm(const vqk_weights *w, const void *x, int32_t x_type,
                   int64_t N, void *y, int32_t y_type, void *workspace,
                   size_t ws_bytes, void *stream);

/* ---- a15: fused MoE decode layer (SwitchGLU + SparseMoeBlock routing) -------
 * mlx-lm's SparseMoeBlock around VQSwitchLinear (restated in
 * bench/decode_ladder.py:107-119 and tests/test_qwen3_5_parity.py:180-205):
 *   ids, w = top_k(softmax(logits[t])), renormalised when norm_topk != 0
 *   y[t] = sum_j w[t, j] * down_e(silu(gate_e(x_t)) * up_e(x_t))
 *          + sigmoid(shared_gate_vec . x_t) * shared(x_t)      (if shared)
 * Routing happens on device from `logits` [T, E] fp32; nothing syncs to the
 * host. gate/up/down are the routed projections (E experts each; gate and up
 * share one format); sh_* are the shared expert (E == 1, same formats), or
 * NULL. topk_ids / topk_w (device, [T, top_k] int32 / fp32) receive the
 * routing when non-NULL.
 *
 * Workspace: vqk_moe_decode_layer_workspace bytes, 256-byte aligned. Its
 * first VQK_MOE_HEADER_BYTES are a header that must be zero before the
 * workspace's first call (hipMemset once when it is allocated, or
 * vqk_moe_layer_reset) and that only layer calls may write afterwards; the
 * rest is scratch whose contents do not matter. One workspace may serve any
 * number of layers, geometries and T, one call at a time: calls sharing a
 * workspace must not overlap. A batch-1 call whose tables fit LDS (a shared
 * expert allowed, E <= 256, d 2 or 4 with 8-12-bit codes, a grid of at most
 * two workgroups per compute unit) runs as ONE launch whose
 * workgroups hand the SwiGLU rows to each other through the header, with a
 * call number kept there between calls. Its waits are bounded (~45 ms): a wait
 * that runs out -- only possible when other work holds the GPU's compute
 * units that long -- makes that call's affected output rows NaN and sets the
 * header's error word, after which every later one-launch call on the
 * workspace returns NaN rows until vqk_moe_layer_reset. No launch ever
 * computes on data that did not arrive. vqk_moe_layer_status reports the
 * error word. */
#define VQK_MOE_HEADER_BYTES 49152u
typedef struct vqk_moe_desc {
    const vqk_weights *gate;
    const vqk_weights *up;
    const vqk_weights *down;
    const vqk_weights *sh_gate;
    const vqk_weights *sh_up;
    const vqk_weights *sh_down;
    const void        *sh_gate_vec;
    int32_t            sh_gate_vec_type;
    int32_t            top_k;
    int32_t            norm_topk;
} vqk_moe_desc;

int vqk_moe_decode_layer_workspace(const vqk_moe_desc *m, int64_t T,
                                   size_t *bytes);
int vqk_moe_decode_layer(const vqk_moe_desc *m, const void *x, int32_t x_type,
                         int64_t T, const float *logits, void *y,
                         int32_t y_type, int32_t *topk_ids, float *topk_w,
                         void *workspace, size_t ws_bytes, void *stream);

/* Header state of a layer workspace (NULL = the current device's
 * no-allocation scratch), with no counterpart in the reference:
 * vqk_moe_layer_status synchronises `stream` and returns VQK_OK, or
 * VQK_EDEVICE with a message when a one-launch call's wait ran out on this
 * workspace; it changes nothing. vqk_moe_layer_reset zeroes the header with a
 * kernel on `stream` (no host synchronisation), clearing the error word and
 * the call number. */
int vqk_moe_layer_status(const void *workspace, void *stream);
int vqk_moe_layer_reset(void *workspace, void *stream);

/* ---- no-allocation variant of vqk_moe_decode_layer ------------------------
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). Same arguments, results and errors as
 * vqk_moe_decode_layer, without the workspace: the layer's scratch is a
 * library-owned device array of VQK_NOALLOC_SCRATCH_BYTES per GPU, taken when
 * the library is loaded on that GPU and held until the process ends. A call
 * whose workspace (vqk_moe_decode_layer_workspace) exceeds it returns
 * VQK_ENOSPACE before any launch (config 4 at T = 64 needs about 19 MB).
 * Every call on one GPU shares that GPU's array: calls that overlap on one
 * GPU (two streams, two threads) race and must be serialised by the caller.
 * The array starts zeroed (static device storage), which its header needs;
 * vqk_moe_layer_status / vqk_moe_layer_reset with workspace NULL act on it.
 * The stream must belong to the current device (else VQK_EINVAL). */
#define VQK_NOALLOC_SCRATCH_BYTES (32u << 20)
int vqk_moe_decode_layer_noalloc(const vqk_moe_desc *m, const void *x, int32_t x_type,
                                 int64_t T, const float *logits, void *y, int32_t y_type,
                                 int32_t *topk_ids, float *topk_w, void *stream);

/* ---- gather-only embeddings: VQEmbedding.__call__ (vq_dense.py:444-502) and
 * VQPLEEmbedding.__call__ (vq_switch.py:5426-5495) ------------------------------
 * out[i, :] = row ids[i] of the table, decoded bit-exactly
 * (fp16(f32(cb[c]) * f32(s))) and converted to out_type (VQK_F16 / VQK_BF16 /
 * VQK_F32; bf16 is one RNE from the fp16 value, like .astype(bfloat16)).
 * The table is a vqk_weights with E == 1 and OUT = table rows; d is 1..16.
 * Code rows: unpacked uint8 / uint16, block-packed uint32 (pack_bits), or the
 * PLE byte stream -- code_type VQK_U8 with pack_bits > 0: code j at bits
 * [j * pack_bits, (j + 1) * pack_bits) of the row's code_cols bytes, LSB
 * first (vq_switch.py:5449-5470). ids: n device VQK_I32 / VQK_I64 entries;
 * an id outside [0, OUT) yields a row of +0. out: [n, IN] device array. */
int vqk_embed_gather(const vqk_weights *w, const void *ids, int32_t id_type,
                     int64_t n, void *out, int32_t out_type, void *stream);

/* ---- capability predicates (1 = this build has a kernel for the shape) -----
 * dense_fits (vq_switch.py:3290-3306), wdec_fits (3505-3514),
 * gemmseg_fits (4469-4507). Same arguments and meaning, answered for the
 * gfx950 kernels of this library. */
int vqk_dense_fits(int64_t K, int64_t IN, int32_t G, int32_t D);
int vqk_wdec_fits(int32_t D, int64_t NSUB, int32_t G, int32_t pack_bits);
int vqk_gemmseg_fits(int32_t D, int64_t K, int32_t G, int32_t pack_bits,
                     int64_t IN);

/* ---- options: the reference's VQ_* dispatch flags as one explicit struct ----
 * The reference steers dispatch with module-global booleans read from the
 * environment at import (vq_switch.py:43-45, 4372, 4421; vq_dense.py:55-102).
 * Here they are arguments: a caller fills a vqk_options (vqk_options_default,
 * or vqk_options_from_env for A/B runs -- the library reads the environment
 * only when asked to) and passes it to the dispatching entry points below.
 *   fused_max_n        VQ_FUSED_MAX_N: routed pairs up to which
 *                      vqk_switch_apply runs the fused GEMV (default 512)
 *   dense_fused_max_n  VQ_DENSE_FUSED_MAX_N: rows up to which vqk_linear_apply
 *                      runs the fused GEMV (default 32)
 *   decode_bf16io      VQ_DECODE_BF16IO: 0 (default) = the fused routed path
 *                      rounds its outputs through fp16 (VQK_VIA_F16); 1 = once
 *                      into y's type, and where the reference's kernel
 *                      stages x as float (unpacked d4 K <= 1024, d8
 *                      K > 1024) bf16 x enters the GEMV unrounded
 *                      (VQK_X_KEEP)
 *   prefill_bf16io     VQ_GEMMSEG_BF16IO: the single output rounding for the
 *                      grouped GEMM path; x is still converted to fp16 on
 *                      stage-in, as the reference's does (vq_switch.py:
 *                      4364-4372). Both flags act on bf16 x only, like the
 *                      reference's _keep_bf16 (vq_switch.py:5306, 5369);
 *                      other x types still round through fp16
 *   crowded_grouped    an extension beyond the reference's dispatch, no VQ_*
 *                      flag: 1 (default) also sends calls whose pairs crowd
 *                      onto few experts (N >= 4 and N >= 2E) to the grouped
 *                      GEMM, which reads each expert's rows once per tile
 *                      instead of once per pair; 0 = the reference's rule
 *                      (N > fused_max_n only). Both paths meet the same
 *                      accuracy bar; the summation order differs. */
typedef struct vqk_options {
    int64_t fused_max_n;
    int64_t dense_fused_max_n;
    int32_t decode_bf16io;
    int32_t prefill_bf16io;
    int32_t crowded_grouped;
} vqk_options;
void vqk_options_default(vqk_options *o);
void vqk_options_from_env(vqk_options *o);

/* VQSwitchLinear.__call__'s dispatch (vq_switch.py:5284-5423): the fused GEMV
 * (vqk_moe_expert_gemv) for at most fused_max_n pairs, else -- or, with
 * crowded_grouped (an extension, see vqk_options), when the pairs crowd onto
 * few experts -- the grouped GEMM (vqk_grouped_gemm), when it takes the
 * module's format. Same arguments as vqk_grouped_gemm plus the
 * options (NULL = defaults); the workspace query returns 0 when the call
 * will run the GEMV. */
int vqk_switch_apply_workspace(const vqk_weights *w, int64_t N, const vqk_options *o,
                               size_t *bytes);
int vqk_switch_apply(const vqk_weights *w, const void *x, int32_t x_type,
                     int64_t T, const uint32_t *eidx, int64_t N, int64_t xkrep,
                     void *y, int32_t y_type, void *workspace, size_t ws_bytes,
                     const vqk_options *o, void *stream);

/* VQLinear.__call__'s dispatch (vq_dense.py:347-441): the fused dense GEMV
 * (vqk_dense_gemv) for at most dense_fused_max_n rows when the shape has a
 * fused kernel (vqk_dense_fits), else the decode-then-GEMM path
 * (vqk_dense_gemm). Outputs are rounded once into y's type, as the
 * reference's dense kernels write x's dtype directly. The GEMV takes d2 / d4
 * x as fp16, as the reference's halfN-staged dense kernels do, and d8 x
 * unrounded (VQK_X_KEEP; the reference has no fused d8 dense kernel and
 * multiplies in x's type). */
int vqk_linear_apply_workspace(const vqk_weights *w, int64_t N, const vqk_options *o,
                               size_t *bytes);
int vqk_linear_apply(const vqk_weights *w, const void *x, int32_t x_type, int64_t N,
                     void *y, int32_t y_type, void *workspace, size_t ws_bytes,
                     const vqk_options *o, void *stream);

/* ---- a14: skipzero row table (skipzero_row_table, vq_switch.py:4958-4973) --
 * rowmask uint8 [E, ceil(OUT / 8)] little bit order -> int32 [E, OUT],
 * compact row of each live (expert, row), -1 = dead. Host memory, like the
 * reference's CPU-stream build. Returns the live-row count in *n_live. */
int vqk_skipzero_row_table_host(const uint8_t *rowmask, int64_t E,
                                int64_t OUT, int32_t *table, int64_t *n_live);

#ifdef __cplusplus
}
#endif

#endif /* VQK_H */
