/* moe_gfx950.h — C-ABI of libmoe_gfx950.so, the MI355X (gfx950, wave64) MoE-block library.
 *
 * Every data pointer is a DEVICE pointer owned by the caller (for example a torch tensor's
 * data_ptr()); `stream` is a hipStream_t passed as void*. Every call is asynchronous on `stream`,
 * allocates no device memory, frees nothing and never synchronises the host; scratch memory
 * comes in through (ws, ws_bytes). One exception to "creates nothing": the first
 * moe_block_forward* call on a device that runs the shared expert beside the routed path creates
 * that device's second stream (default priority, non-blocking) and two events, kept until the
 * process ends. That is a call of 7 or more tokens, except where the step folds the shared expert
 * into its own launches (up to 256 tokens with Q4_K routed weights, bf16 shared weights,
 * H % 2048 == 0 and I_s % 256 == 0: one stream). moe_block_forward_w_noalloc never forks. Routing values never
 * travel to the host (specification/11-moe-block.md §11.7: the block is computable with zero
 * host-visible routing values).
 *
 * Return value: MOE_OK (0) or a negative MOE_E_* code; moe_last_error() then returns a
 * thread-local description. Nothing throws across the ABI. Results are deterministic: no float
 * atomics write any returned tensor, so equal inputs give equal bits.
 *
 * The reference has no C-ABI: its MoE step is the Python call surface
 *   engine/block_forward.py:614-681  moe_router / moe_shared / moe_routed / moe_block
 *   engine/m3_forward.py:430-476     moe_block(g, E, layer)
 *   speccheck/moe_ref.py:318-533     route / expert_gather / shared_expert / moe_block
 * and its device work ran as separate processes (engine/device_arm.py:417-463). Each entry point
 * below names the reference function it replaces.
 */
#ifndef MOE_GFX950_H
#define MOE_GFX950_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOE_ABI_VERSION 3

enum {
  MOE_OK = 0,
  MOE_E_ARG = -1,          /* bad pointer, shape or enum                                     */
  MOE_E_FORMAT = -2,       /* weight format not supported for this operand                   */
  MOE_E_HIP = -3,          /* a HIP runtime call failed (text in moe_last_error)             */
  MOE_E_WORKSPACE = -4,    /* ws_bytes smaller than moe_workspace_bytes() asks for            */
  MOE_E_UNSUPPORTED = -5   /* geometry outside what the kernels are built for                */
};

/* dtypes of activations / outputs */
enum { MOE_DT_F32 = 0, MOE_DT_BF16 = 1 };

/* weight formats: ggml_type ids (tools/gguf_reader.py:10-51 block table). Routed gate_up: Q4_K,
 * Q6_K or BF16; routed down: Q4_K, Q5_K (the shipped artifact's down in 37 of its 40 layers,
 * engine/README.md:33,115), Q6_K or BF16; shared expert: BF16 or Q8_0 (the artifact's
 * ffn_*_shexp); lm_head table: Q6_K, Q8_0 or BF16; moe_dequant: Q4_K, Q5_K, Q6_K. */
enum { MOE_FMT_Q8_0 = 8, MOE_FMT_Q4_K = 12, MOE_FMT_Q5_K = 13, MOE_FMT_Q6_K = 14, MOE_FMT_BF16 = 30 };

/* expert contraction path: GEMV = fused decode + f32 GEMV; MFMA = tiles decoded to f16 in LDS on
 * MFMA (f32 accumulation); MFMA_BF16 = the same with bf16 operands (8 significant bits instead of
 * 11; same MFMA rate). MFMA_BF16 is OUTSIDE the block-output bar that AUTO, GEMV, MFMA and
 * GEMV_MULTI meet (max-abs 2e-3 / rel 1e-2 against the f32 oracle): its outputs land ~3e-3 from the
 * oracle (~4e-4 for MFMA), and its test holds it to 8e-3. AUTO never picks it; it is there only for
 * a caller that asks for bf16 operands by name. A single-token moe_block_forward on the GEMV path
 * runs one persistent launch on devices with >= 256 CUs; GEMV_MULTI forces the three-launch form
 * of the same arithmetic (any CU count). */
enum { MOE_PATH_AUTO = 0, MOE_PATH_GEMV = 1, MOE_PATH_MFMA = 2, MOE_PATH_MFMA_BF16 = 3,
       MOE_PATH_GEMV_MULTI = 4 };

int moe_abi_version(void);
const char *moe_last_error(void);

/* Scratch bytes moe_block_forward / moe_experts / moe_sort_permute / moe_router_topk need for a
 * T-token step of this geometry (an upper bound for every path). */
size_t moe_workspace_bytes(int T, int H, int I, int E, int K, int I_s);

/* Scratch bytes moe_router_topk can use for T tokens (the sync words, the logits when
 * logits_bf16 is NULL, and the int8 matrix-core R1's row metadata and router digit planes).
 * No reference counterpart: a workspace of this size (or of moe_workspace_bytes) lets R1 at
 * T > 256 run on the int8 matrix cores; a smaller one, or none, keeps it on the f64 matrix cores.
 * The logits are the same bits either way. */
size_t moe_router_workspace_bytes(int T, int H, int E);

/* Bit-exact super-block decode: n_elts elements of `fmt` blocks -> f32 or bf16 (RNE of the exact
 * f32 value). Replaces tools/gguf_reader.py:248-268 (_deq_q4_k), :271-296 (_deq_q5_k),
 * :299-322 (_deq_q6_k) and tools/gguf_fast_dequant.py:87-152 (dequant_np). n_elts % 256 == 0. */
int moe_dequant(const void *blocks, int fmt, int64_t n_elts, void *out, int out_dtype,
                void *stream);

/* R1-R5 for T tokens. Replaces speccheck/moe_ref.py:318-363 (route) and
 * engine/block_forward.py:614-636 (moe_router); engine/m3_forward.py:443-446.
 *   R1 logits[t,e] = bf16 of the correctly rounded sum_j x[t,j]*W[e,j] (+ logit_bias[e])
 *   R2 probs = softmax over E in f32; R3 top-K with torch CPU's tie order;
 *   R4 w_f32 = renormalised top-K probs; R5 w_bf16 = bf16(w_f32).
 * x: [T,H] f32 or bf16; w_router: [E,H] in w_dtype: MOE_DT_BF16, or MOE_DT_F32 (the shipped
 * artifact's F32 ffn_gate_inp, engine/block_forward.py:221-231; x*W products stay exact in f64,
 * so R1 is correctly rounded either way); logit_bias: [E] f32 or NULL.
 * logits_bf16 [T,E], probs [T,E] may be NULL; topk_ids [T,K] int32; w_f32, w_bf16 [T,K].
 * Limits: H % 512 == 0, E <= 256, K <= 16, K * 64 > E (torch's nth_element branch).
 * ws: NULL when logits_bf16 is given, else at least the sync words and the logits; with
 * moe_router_workspace_bytes(T, H, E) bytes, R1 at T > 256 runs on the int8 matrix cores. */
int moe_router_topk(const void *x, int x_dtype, const void *w_router, int w_dtype,
                    const float *logit_bias, int T, int H, int E, int K, void *logits_bf16, float *probs,
                    int32_t *topk_ids, float *w_f32, void *w_bf16, void *ws, size_t ws_bytes,
                    void *stream);

/* Stable token->expert grouping: pairs p = t*K + k sorted by expert id, ties in p order,
 * bit-exact vs torch.argsort(ids.flatten(), stable=True). Replaces the grouping in
 * speccheck/moe_ref.py:433-439 and engine/m3_forward.py:448-452.
 * expert_offsets [E+1]; sorted_pairs [T*K] (value p); pair_pos [T*K] (inverse permutation);
 * hit_list [E+1] = n_hit, then the hit expert ids ascending. ws: as every entry point's, its
 * first 512 KiB are the sync words (left untouched); T*K > 64 needs scratch after them. */
int moe_sort_permute(const int32_t *topk_ids, int T, int K, int E, int32_t *expert_offsets,
                     int32_t *sorted_pairs, int32_t *pair_pos, int32_t *hit_list, void *ws,
                     size_t ws_bytes, void *stream);

/* The K routed SwiGLU experts of every token, grouped so each hit expert's weights are read once
 * per step. Replaces speccheck/moe_ref.py:367-451 (_expert_apply, expert_gather) and
 * engine/m3_forward.py:452-463. gate_up_q: [E][2I rows][H/256 blocks], gate rows first
 * (spec §11.4), when up_q is NULL; else gate_up_q holds the gate rows [E][I rows][H/256 blocks]
 * and up_q the up rows in the same layout (the artifact's separate ffn_gate_exps and
 * ffn_up_exps). down_q: [E][H rows][I/256 blocks]. y [T*K, H] f32 in sorted-pair order
 * (expert_raw before the routing weight). path: GEMV = fused dequant + f32 GEMV (decode),
 * MFMA / MFMA_BF16 = tiles dequantised to f16 / bf16 in LDS, contracted on MFMA (prefill);
 * AUTO picks GEMV for T <= 6 with Q4_K gate_up and Q4_K / Q5_K / Q6_K down, MFMA otherwise.
 * Formats the chosen path cannot read are refused before anything is queued. */
int moe_experts(const void *x, int x_dtype, const void *gate_up_q, const void *up_q, int gate_up_fmt,
                const void *down_q, int down_fmt, const int32_t *expert_offsets,
                const int32_t *sorted_pairs, const int32_t *hit_list, int T, int H, int I, int E,
                int K, int path, float *y, void *ws, size_t ws_bytes, void *stream);

/* Shared expert and its scalar sigmoid gate. Replaces speccheck/moe_ref.py:480-495,
 * engine/block_forward.py:639-649 and engine/m3_forward.py:436-442.
 * w_gate, w_up: [I_s,H]; w_down: [H,I_s], in shared_fmt: MOE_FMT_BF16, or MOE_FMT_Q8_0 (GGUF
 * rows of 34-byte blocks, the artifact's ffn_*_shexp; H and I_s multiples of 256, 16-byte
 * aligned tensors); w_scalar_gate: [H] in
 * gate_dtype (MOE_DT_BF16, or MOE_DT_F32 as the artifact's ffn_gate_inp_shexp).
 * shared_raw [T,H] = down(silu(gate x) * up x); gate_prob [T] = sigmoid(w_scalar_gate . x). */
int moe_shared_expert(const void *x, int x_dtype, const void *w_gate, const void *w_up,
                      const void *w_down, int shared_fmt, const void *w_scalar_gate, int gate_dtype,
                      int T, int H, int I_s, int path, float *shared_raw, float *gate_prob, void *ws,
                      size_t ws_bytes, void *stream);

/* Top-K weighted combine, ascending expert id, weight reached by rank, plus the gated shared
 * expert. Replaces speccheck/moe_ref.py:452-476, :516-518 and engine/block_forward.py:664-667,
 * :680. y: [T*K,H] sorted order; w_bf16 [T,K]; out [T,H] f32; routed_sum, shared_out [T,H] and
 * expert_raw [T,K,H] (slot order) are optional (NULL). */
int moe_combine(const float *y, const int32_t *pair_pos, const int32_t *topk_ids,
                const void *w_bf16, const float *shared_raw, const float *gate_prob, int T, int K,
                int H, float *out, float *routed_sum, float *shared_out, float *expert_raw,
                void *stream);

/* The whole block in one stream-ordered call. Replaces speccheck/moe_ref.py:499-533 (moe_block),
 * engine/block_forward.py:670-681 and engine/m3_forward.py:430-476.
 * norm_w [H] f32 (optional): the block input is then the post-attention RMSNorm of x, Form A with
 * the artifact's (1+w) already in norm_w (engine/m3_forward.py:303-307, :732-733):
 * (x * f32(1/sqrt(mean(x^2) + norm_eps))) * norm_w, the scale evaluated in f64 and rounded once;
 * NULL: x is the block input as given. out = residual + MoE(input) when `residual` [T,H] f32 is
 * given (the decoder layer's own residual add, engine/m3_forward.py:737; out may alias residual
 * and x), else MoE(input). Stage outputs other than `out` may be NULL; expert_raw is [T,K,H] in
 * slot order. A single token with K = 8 and Q4_K gate_up runs the single-launch decode layer
 * (the norm fused into it) on devices with >= 256 CUs, else the three-launch decode path. */
int moe_block_forward(const void *x, int x_dtype, int T, int H, int I, int E, int K, int I_s,
                      const float *norm_w, float norm_eps, const void *w_router, const float *logit_bias, const void *gate_up_q,
                      int gate_up_fmt, const void *down_q, int down_fmt, const void *ws_gate,
                      const void *ws_up, const void *ws_down, const void *ws_scalar_gate,
                      int path, const float *residual, float *out, void *logits_bf16,
                      int32_t *topk_ids, void *topk_w_bf16, float *topk_w_f32,
                      float *routed_sum, float *shared_out, float *gate_prob, float *expert_raw,
                      void *ws, size_t ws_bytes, void *stream);

/* One layer's MoE weights with their formats: what the layer loop of engine/m3_forward.py:714-737
 * reads per layer (E.read roles, engine/m3_forward.py:235-283), in the widths a caller holds them:
 * the synthetic configs' bf16 router / fused gate_up / bf16 shared expert, or the shipped
 * artifact's F32 router and scalar gate, separate gate and up tensors and Q5_K / Q6_K down
 * (engine/README.md:33, engine/block_forward.py:221-231). */
typedef struct moe_layer_weights {
  const void *w_router;          /* [E,H] */
  int router_dtype;              /* MOE_DT_BF16 or MOE_DT_F32 */
  const float *logit_bias;       /* [E] f32 or NULL */
  const void *gate_q;            /* fused gate_up [E][2I rows] (up_q NULL) or gate [E][I rows] */
  const void *up_q;              /* up [E][I rows], or NULL */
  int gate_up_fmt;               /* MOE_FMT_Q4_K (also Q6_K / BF16 off the decode paths) */
  const void *down_q;            /* [E][H rows] */
  int down_fmt;                  /* MOE_FMT_Q4_K, Q5_K, Q6_K (BF16 off the decode paths) */
  const void *ws_gate, *ws_up;   /* [I_s,H] */
  const void *ws_down;           /* [H,I_s] */
  int shared_fmt;                /* MOE_FMT_BF16 or MOE_FMT_Q8_0 */
  const void *ws_scalar_gate;    /* [H] */
  int scalar_gate_dtype;         /* MOE_DT_BF16 or MOE_DT_F32 */
  const float *norm_w;           /* [H] f32 post-attention norm weight, or NULL */
} moe_layer_weights;

/* moe_block_forward over a moe_layer_weights (w; norm_w and every weight pointer from there) and an
 * optional next-layer hint (next: as moe_block_forward_prefetch, the router rows and norm weight of
 * a bf16-router next layer). Same outputs, limits and errors as moe_block_forward. The
 * single-launch decode layer takes a bf16 or f32 router and scalar gate, Q4_K gate/up (fused or
 * split), Q4_K, Q5_K or Q6_K down, and a bf16 or Q8_0 shared expert. Of `next` only the router
 * rows (w_router, router_dtype: bf16 or f32) and norm_w are read, as the L2 warm-up hint.
 * Replaces engine/m3_forward.py:430-476 and engine/block_forward.py:670-681 on the policy-A
 * weights (engine/block_forward.py:211-231). */
int moe_block_forward_w(const void *x, int x_dtype, int T, int H, int I, int E, int K, int I_s,
                        const moe_layer_weights *w, float norm_eps, int path, const float *residual,
                        float *out, void *logits_bf16, int32_t *topk_ids, void *topk_w_bf16,
                        float *topk_w_f32, float *routed_sum, float *shared_out, float *gate_prob,
                        float *expert_raw, void *ws, size_t ws_bytes, void *stream,
                        const moe_layer_weights *next);

/* The weights of the layer that the same stream runs next that its routing waits on: its router
 * rows and its post-attention norm weight (shapes as in moe_block_forward). The next layer's
 * shared expert is not named: its rows have slack in that layer (requested at its first barrier,
 * off the routing chain), and warming them here measured slower (the extra 6.3 MB of misses
 * delay this layer's last exchange more than they save). */
typedef struct moe_next_layer {
  const void *w_router;         /* [E,H] bf16 */
  const float *norm_w;          /* [H] f32, or NULL when the next call passes no norm weight */
} moe_next_layer;

/* moe_block_forward with a hint: `next` (may be NULL) names the next layer's router rows and norm
 * weight. The single-launch decode layer then reads them at the end of its run (each workgroup its
 * own router rows), so that they come from the L2 of the same XCD instead of HBM. Other paths
 * ignore the hint. Results are identical with or without it.
 * Same arguments, limits and errors as moe_block_forward otherwise. Replaces, like
 * moe_block_forward, engine/m3_forward.py:430-476 in its layer loop (engine/m3_forward.py:714-737),
 * where the next layer's weights are known ahead of its input. */
int moe_block_forward_prefetch(const void *x, int x_dtype, int T, int H, int I, int E, int K, int I_s,
                               const float *norm_w, float norm_eps, const void *w_router,
                               const float *logit_bias, const void *gate_up_q, int gate_up_fmt,
                               const void *down_q, int down_fmt, const void *ws_gate,
                               const void *ws_up, const void *ws_down, const void *ws_scalar_gate,
                               int path, const float *residual, float *out, void *logits_bf16,
                               int32_t *topk_ids, void *topk_w_bf16, float *topk_w_f32,
                               float *routed_sum, float *shared_out, float *gate_prob,
                               float *expert_raw, void *ws, size_t ws_bytes, void *stream,
                               const moe_next_layer *next);

/* moe_block_forward_w for callers that cannot allocate (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). No counterpart in the reference. Same arguments,
 * outputs, limits and errors as moe_block_forward_w, without (ws, ws_bytes): the scratch is a
 * static device array of MOE_NOALLOC_SCRATCH_BYTES inside the library, one per device, held until
 * the process ends. A step needing more scratch than that (moe_workspace_bytes(T, ...) >
 * MOE_NOALLOC_SCRATCH_BYTES: above MOE_NOALLOC_MAX_T tokens at the model's geometry) is refused
 * with MOE_E_WORKSPACE before anything is queued. The call allocates nothing: no hipMalloc, no
 * stream or event (the shared expert runs on `stream`, where moe_block_forward_w would fork a
 * second stream from 7 tokens on; the bits are the same). The first call on a device clears the
 * array's sync words with a fill launch on `stream`. Every call on one device shares that device's
 * array: calls that overlap on one GPU (two streams, two threads) race and must be ordered by
 * the caller. */
#define MOE_NOALLOC_SCRATCH_BYTES (16u << 20)
#define MOE_NOALLOC_MAX_T 120  /* the largest T whose moe_workspace_bytes fits, at H=2048 I=512 E=256 K=8 I_s=512 */
int moe_block_forward_w_noalloc(const void *x, int x_dtype, int T, int H, int I, int E, int K, int I_s,
                                const moe_layer_weights *w, float norm_eps, int path,
                                const float *residual, float *out, void *logits_bf16,
                                int32_t *topk_ids, void *topk_w_bf16, float *topk_w_f32,
                                float *routed_sum, float *shared_out, float *gate_prob,
                                float *expert_raw, void *stream, const moe_layer_weights *next);

/* Untied lm_head GEMV: logits[b, j] = sum_k h[b, k] * W[row_j, k] in f32 for b < B (1..8) and
 * j < n_rows, with row_j = j (dense: row_ids NULL, n_rows <= V) or row_j = row_ids[j] (gather; an
 * id outside [0, V) gives NaN for that output). h: [B, H] f32 or bf16 (h_dtype); W: V rows of H
 * in w_fmt: MOE_FMT_Q6_K (H/256 x 210 B per row: the shipped artifact's output.weight,
 * engine/README.md:33), MOE_FMT_Q8_0 (H/32 x 34 B) or MOE_FMT_BF16 (H x 2 B); W 16-byte aligned.
 * logits: [B, n_rows] f32. Limits: H == 2048. Tokens go in passes of up to 4, each reading the
 * table once. Results are f32 dots in this kernel's association order: they lie within the
 * reference's band gamma_n * sum_k |h_k w_k| (n = K-1 for exact products, 2K-1 otherwise;
 * prototype/lm_head/gate.py:214-240) of the exact dot. Replaces prototype/lm_head/
 * lm_head_kernels.h:474-512 (lmh_dot_batch) as launched by prototype/lm_head/lm_head.hip:51. */
int moe_lm_head(const void *h, int h_dtype, int B, int H, const void *w, int w_fmt, int64_t V,
                const int32_t *row_ids, int64_t n_rows, float *logits, void *stream);

/* The workspace's status word, stream-ordered: *status (a device int32 the caller owns) receives
 * the bits recorded since the last call, and the word is cleared. Bit MOE_STATUS_SPIN_TIMEOUT: a
 * bounded wait of the single-launch decode layer gave up (its workgroups were not all co-resident,
 * or not placed on the XCDs round robin as it assumes); the output rows of every workgroup that
 * gave up are NaN and the rest of that call's outputs are unspecified. Bit MOE_STATUS_SYNC_STATE:
 * a block-arrival counter of the single-launch router (8 to 256 tokens) held a count its launch
 * cannot produce (a workspace that skipped moe_workspace_init, or two calls overlapping on one
 * workspace); that call's logits, ids, weights and block outputs are unspecified (every stage of
 * the launch still runs once, so the grouped GEMMs after it stay in bounds), and
 * moe_workspace_init restores the counters. No host synchronisation:
 * read *status after the stream reaches it. No counterpart in the reference (its device work ran
 * in fresh processes and reported through their exit status, engine/device_arm.py:417-463). */
#define MOE_STATUS_WORD 3              /* int32 index of the status word in the workspace */
#define MOE_STATUS_SPIN_TIMEOUT 1
#define MOE_STATUS_SYNC_STATE 2
/* Test hook: while the workspace's int32 word MOE_TEST_HOOK_WORD is non-zero, every bounded wait
 * of the single-launch decode layer completes as usual and then reports a timeout, so a caller's
 * handling of the status and the NaN rows can be exercised without a real timeout. Zero in normal
 * use (moe_workspace_init clears it). */
#define MOE_TEST_HOOK_WORD 4
int moe_workspace_status(void *ws, size_t ws_bytes, int32_t *status, void *stream);

/* Zero the workspace's device-side sync words (its first 512 KiB: status bits, the single-launch
 * decode layer's per-role launch counts and its two exchange buffers; one short fill launch).
 * Call once after allocating a workspace, before its first use by moe_block_forward /
 * moe_experts / moe_shared_expert / moe_router_topk; a workspace zeroed by other means is the
 * same starting state. Every call leaves the words valid for the next.
 * Calls sharing one workspace must be ordered on one stream. No counterpart in the reference (its
 * device work ran in fresh processes). */
int moe_workspace_init(void *ws, size_t ws_bytes, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* MOE_GFX950_H */
