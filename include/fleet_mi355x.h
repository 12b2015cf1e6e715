/* fleet_mi355x.h - C ABI of the MI355X (gfx950) batch-1 DeepSeek-V2-Lite decode path.
 *
 * The reference drives its decode through a Python plan -> mirage runtime boundary:
 *   mi.PersistentKernel(...), mpk.attach_input / mpk.<op>_layer / kn_graph.register_task,
 *   mpk.compile(), mpk()                          (fleet/build_graph.py:36-46, 478-528, 561-593;
 *                                                  harness/run_fleet.py:551-593)
 * and a per-kernel launcher for its kernel suite (fleet/tasks/kernel_tests_mi300.cu:1-47).
 * This header is that boundary as a C ABI: plain pointers and sizes, no torch types. The host
 * (fleet/build_graph.py's counterpart, through ctypes) owns every device buffer of the model and
 * hands raw device pointers in a task table (the plan's calls, one fx_stage each); the library
 * owns only its error flag and timing slots.
 *
 * Errors: every entry returns 0 on success or a nonzero FX_E_* code; fx_last_error() returns the
 * message of the last failure on that context (mirrors the suite's exit codes,
 * kernel_tests_mi300.cu:46-47, and the plan asserts run before launch, harness/run_fleet.py:507-513).
 * Threading: one host thread per context; fx_run returns after every iteration has finished, as
 * mpk() does (harness/run_fleet.py:590-593).
 */
#ifndef FLEET_MI355X_H
#define FLEET_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FX_ABI_VERSION 4

/* ---- error codes ---------------------------------------------------------------------------- */
#define FX_OK 0
#define FX_E_HIP 1         /* a HIP runtime call failed */
#define FX_E_ARG 2         /* an argument or a plan entry is invalid (checked before launch) */
#define FX_E_DEVICE 3      /* the device is not a gfx950 with the expected layout */
#define FX_E_STATE 4       /* call out of order (no plan loaded, ...) */

/* ---- dataflow between stages ------------------------------------------------------------------
 * There is no barrier between stages. Every activation one stage hands to another travels as
 * tagged packets: 8 bytes = a 32-bit payload (two bf16, element 2i in the low half, or one f32)
 * and the 32-bit tag of the producing stage. A consumer polls exactly the packets it needs until
 * their tags equal the producer's tag, so a stage starts as soon as its own inputs exist (and
 * issues its weight loads before it polls). Tags: stage s of iteration i of a launch with
 * epoch0 E writes tag E + i * n_stages + s + 1; fx_stage.src[k] names the stage (index in the
 * table, negative = that many stages back, i.e. the previous iteration) whose tag input k
 * carries. Buffers marked "packets" below hold 8 bytes per value pair (bf16) or per value (f32)
 * and must be zeroed before first use (tag 0 is never produced). Plain buffers (caches, partials,
 * dumps) are ordinary arrays. */

/* ---- operators of the task table --------------------------------------------------------------
 * One per plan call (fleet/graph_plan.py OUTPUT_ARGS names in brackets). Every device pointer is
 * a bf16 (uint16) array unless marked f32 / i32 / i64 / packets. 256 workers: worker w is workgroup
 * w, on XCD w % 8, rank w / 8 of its XCD's 32. */
enum fx_op {
  /* [linear_gemv_layer] out[n] = bf16(dot(w[n], xin) (+ res[n])) for n < n_rows; K = k; rows in
   * groups of 4 split over all workers. Input xin by in_kind: FX_IN_VEC x (packets, src[0]);
   * FX_IN_EMBED w_embed(aux0)[token], token = tokens(aux4 i64)[step] inside the prompt, else the
   * argmax of amax(aux3 packets f32, src[1]), stored by worker 0 to tokens[step].
   * FX_F_NORM: xin := rmsnorm(xin, w_norm). FX_F_RESIDUAL: res (packets, src[2]);
   * FX_F_RES_EMBED: the residual is w_embed(aux0)[token of this iteration].
   * FX_F_OUT_LL: out is packets, else a plain bf16 array. FX_F_ARGMAX: per-worker (max, index) of
   * the bf16 outputs to amax(aux3 packets f32 [2 * 256]). */
  FX_OP_GEMV = 1,
  /* [mla_prep_layer] qkva(x packets, src[0]) -> cache rows c_kv(aux0)[step], k_pe(aux1)[step]
   * (plain), ql_nope(out packets) [nh, d_c], q_pe(aux2 packets) [nh, d_r], and per XCD a packet copy
   * of the cache row crow(aux5 packets) [8][d_c + d_r]; w = W_uk [nh, d_n, d_c]; w_norm =
   * kv_a_layernorm weight; cos(aux3), sin(aux4) [s_max, d_r]. XCD x owns heads 2x, 2x + 1. */
  FX_OP_MLA_PREP = 2,
  /* [mla_attend_layer] ql_nope(x packets), q_pe(aux2 packets), crow(aux5 packets) (src[0] each),
   * caches c_kv(aux0), k_pe(aux1) -> partials(out f32) [n_splits, nh, prow] (o, then lse at d_c) for
   * the live splits, split j on rank j % 32 of each XCD; each worker then publishes a done packet
   * done(aux6 packets f32) [8][32]. */
  FX_OP_MLA_ATTEND = 3,
  /* [mla_merge_uv_layer] the LSE merge of head h's live partials (x f32, after done(aux6), src[0])
   * into bf16 o, then attn(out packets)[h*d_v+v] = bf16(dot(o, W_uv(w)[h][v])), d_v in the d_n field;
   * ranks 0..15 / 16..31 of XCD x take heads 2x / 2x + 1, 8 rows each; o to o_merged(aux4) (plain). */
  FX_OP_MLA_MERGE_UV = 4,
  /* [moe_router_layer] h = rmsnorm(x_res(x packets, src[0]), w_norm); logits(out packets f32)[e] =
   * dot(W_gate(w)[e], h) for e < n_rows, row e on worker e. */
  FX_OP_MOE_ROUTER = 5,
  /* [gang_moe_w13_gemv_layer (+ moe_router_layer)] every worker takes pair groups of every slot's
   * expert (slot s: the top-k routed experts, then the n_forced shared experts E, E+1), shared slots
   * first; h = rmsnorm(x_res(x packets, src[1])); act8(out packets)[slot][i] = bf16(silu(bf16(W13(w)[e][i] h))
   * * bf16(W13[e][I+i] h)), I = n_rows; expert ids from logits(aux0 packets f32, src[0]). FX_F_ROUTER:
   * the stage itself computes logits[e] = dot(W_gate(res)[e], h) on worker e and reads them back.
   * Worker 0 stores topk_w(aux1 f32), routing(aux2 i32), mask(aux3 i32), logits(aux4 f32), h(aux6),
   * sel(aux7 i32 [8]) and route_log(aux5 i32 [prow][aux_i1][n_slots]) at row step - (n_prompt - 1) when
   * that row is in [0, prow); aux_i0 = E. */
  FX_OP_MOE_W13 = 6,
  /* [gang_moe_w2_linear_layer + moe_mul_sum_add_layer] out8[s][n] = bf16(dot(W2(w)[e_s][n],
   * act8(x packets, src[0])[s])) for every slot s, experts from logits(aux0 packets f32, src[1]);
   * x_new(out packets)[n] = bf16(x_res(res packets, src[2])[n] + sum_s out8[s][n] * topk_w[s])
   * (slot order); n_rows = H rows in groups of 8 per worker, k = I; out8 also to aux1 when non-NULL. */
  FX_OP_MOE_W2 = 7,
  /* [gang_linear_silu_layer] h = rmsnorm(x_res(x packets, src[0]), w_norm); act(out packets)[i] =
   * bf16(silu(bf16(w[i] h)) * bf16(w[I+i] h)) for i < n_rows (= I); h to aux6 when non-NULL. */
  FX_OP_DENSE_GU = 9,
  /* [argmax_reduce_layer] tokens(aux4 i64)[step + 1] = argmax from amax(aux3 packets f32, src[0]). */
  FX_OP_ARGMAX = 10,
};

/* GEMV input kinds */
#define FX_IN_VEC 0
#define FX_IN_EMBED 1

/* flags */
#define FX_F_NORM 1u
#define FX_F_RESIDUAL 2u
#define FX_F_ARGMAX 8u
#define FX_F_HEAD 16u      /* the stage belongs to the head: skipped while step + 1 < n_prompt */
#define FX_F_OUT_LL 32u    /* output as packets */
#define FX_F_RES_EMBED 64u /* residual = the embedding row of this iteration's token */
#define FX_F_ROUTER 128u   /* MOE_W13 computes the router itself (W_gate in res) */
#define FX_F_FP8 256u      /* MOE_W13 / MOE_W2, or the LM head GEMV (FX_F_ARGMAX) of a plan whose expert stages
                            * are FP8: w is FP8 (OCP e4m3fn codes [rows][k], then one f32 scale per row) */
#define FX_F_MFMA 512u     /* MLA_ATTEND / MLA_MERGE_UV: the matrix-core attention. Split j runs on worker
                            * j % 256 for all heads (tiles of 32 positions; scores and value products on
                            * v_mfma_f32_16x16x32_bf16); done(aux6) holds one packet per worker, the merge
                            * waits for workers 0 .. min(live splits, 256) - 1 and runs on ranks 16..31 of
                            * every XCD (workers 128..255): ranks 16..23 / 24..31 of XCD x take head 2x /
                            * 2x + 1, 16 W_uv rows each. MLA_MERGE_UV aux7 (optional, [n_rows][d_c] packets):
                            * with 9..176 live splits each of a head's 8 workers merges 64 columns and
                            * they exchange them there (XCD-local) before W_uv */

#define FX_F_XLOCAL 1024u  /* MLA_PREP: every reader of its packets runs on the producing XCD (the VALU
                            * attention: XCD x owns heads 2x, 2x + 1), so they are stored XCD-local (sc0)
                            * instead of device-coherent (sc1) */
#define FX_F_XCD 2048u     /* the single-XCD matrix-core attention. MLA_ATTEND: the stage does nothing.
                            * MLA_MERGE_UV: the attention of every head and its merge on the 32 workers of
                            * XCD 7 (split j on rank j % 32, rank r merges head r / 2 and W_uv rows
                            * 64 (r % 2) ..); partials (x) and done packets (aux6, one per rank) stay in
                            * that XCD's L2. The attention's operands ride in the merge's spare fields:
                            * aux3 = ql_nope packets, aux0 c_kv, aux1 k_pe, aux2 q_pe packets, aux5 crow
                            * packets, scale, s_max; src[0] = their producer */
#define FX_F_SKIP_XCD 4096u /* GEMV: rows split over the workers of XCDs 0..6 only (XCD 7 runs the
                            * single-XCD attention just before) */
#define FX_F_LOW16 16384u  /* GEMV: rows split over ranks 0..15 of every XCD (workers 0..127) only: the
                            * matrix-core attention's merge runs on ranks 16..31 just before, and those
                            * workers go on to the expert stage's first loads instead (FX_F_PAIR) */
#define FX_F_PAIR 8192u    /* GEMV followed by a MOE_W13 stage: the persistent kernel runs the two as one
                            * operator that issues the expert stage's first weight loads (its shared
                            * groups, router row, norm weights) before the GEMV's own, so they stream while
                            * the GEMV waits for its input. The kernel suite's one-stage launches ignore
                            * the flag. Not with FX_F_ARGMAX, FX_F_HEAD or FX_F_SKIP_XCD */

/* One entry of the task table: one operator of the plan (fleet/graph_plan.py Call). */
typedef struct fx_stage {
  int32_t op, flags, in_kind;
  int32_t layer;      /* decoder layer (route_log row: layer - 1), -1 outside the layers */
  int32_t n_rows;     /* GEMV/DENSE_GU rows; heads for MLA ops; E for the router; H for W2 */
  int32_t k;          /* reduction width (H, or I for W2 / down) */
  int32_t n_slots;    /* MoE slots: topk + forced (8) */
  int32_t topk, n_forced, split, n_splits;
  int32_t d_c, d_r, d_n, prow;
  int32_t s_max, aux_i0, aux_i1;
  int32_t src[4];     /* producing stage of each packet input (see "dataflow") */
  float eps, scale, scaling, aux_f;
  uint64_t w, x, w_norm, res, out;
  uint64_t aux[8];
} fx_stage;

/* ---- context ---------------------------------------------------------------------------------- */
typedef struct fx_ctx fx_ctx;

/* Replaces mi.PersistentKernel(...) (fleet/build_graph.py:583-589): binds a device, checks it is a
 * gfx950 with 256 CUs in 8 XCDs, allocates the error flag and timing slots. */
int fx_create(int device, fx_ctx** out);
int fx_destroy(fx_ctx* ctx);
const char* fx_last_error(fx_ctx* ctx);
int fx_abi_version(void);

/* Device facts: CUs, XCDs, workers (one per CU), LDS per workgroup. */
int fx_device_info(fx_ctx* ctx, int32_t* cus, int32_t* xcds, int32_t* workers, int32_t* lds_bytes);

/* ---- memory (for hosts without torch: the ctypes runtime allocates through these) ------------- */
int fx_malloc(fx_ctx* ctx, size_t nbytes, void** dptr);
int fx_free(fx_ctx* ctx, void* dptr);
int fx_memcpy_htod(fx_ctx* ctx, void* dst, const void* src, size_t nbytes);
int fx_memcpy_dtoh(fx_ctx* ctx, void* dst, const void* src, size_t nbytes);
int fx_memcpy_dtod(fx_ctx* ctx, void* dst, const void* src, size_t nbytes);
int fx_memset(fx_ctx* ctx, void* dst, int value, size_t nbytes);
int fx_synchronize(fx_ctx* ctx);

/* ---- plan and run ----------------------------------------------------------------------------- */
/* Replaces mpk.compile() (the codegen + JIT of the worker switch, harness/run_fleet.py:556): the
 * task table is validated on the host (shapes, pointers, packet sources) and uploaded. */
int fx_load_plan(fx_ctx* ctx, const fx_stage* stages, int32_t n_stages, const fx_stage* epilogue,
                 int32_t n_epilogue);

/* Replaces mpk() (harness/run_fleet.py:590-593): one persistent launch that runs `iters` decode
 * iterations at positions step0 .. step0 + iters - 1. tokens (int64 [>= step0 + iters + 1]) holds the
 * prompt in [0, n_prompt); iteration i reads tokens[step0 + i] and, when step0 + i + 1 >= n_prompt,
 * the head's argmax is stored to tokens[step0 + i + 1]. stream: a hipStream_t or NULL. n_prompt >= 1.
 * A launch whose step0 lies past the prompt (step0 >= n_prompt) reads its first token from the previous
 * iteration's argmax, so it must continue the previous launch of the same plan (step0 == that launch's
 * step0 + iters); any other such launch fails with FX_E_ARG. */
int fx_run(fx_ctx* ctx, int32_t iters, int32_t step0, int32_t n_prompt, int64_t* tokens, void* stream);

/* fx_run in two halves, so that launches can be queued back to back: fx_launch enqueues the
 * persistent launch on `stream` and returns (no host wait); fx_finish waits for the stream and
 * reports a wait that timed out inside any launch since the last fx_finish. fx_run = both. A launch
 * whose iterations all lie inside the prompt (step0 + iters < n_prompt: the head never runs) uses
 * the kernel symbol fx_prefill, every other launch fx_persistent (the same code). iters is at most
 * FX_MAX_ITERS. Tags are 32-bit and never reused: a launch that would exhaust them fails with
 * FX_E_STATE (after about 2^32 / n_stages iterations of one context). */
#define FX_MAX_ITERS 65536
int fx_launch(fx_ctx* ctx, int32_t iters, int32_t step0, int32_t n_prompt, int64_t* tokens, void* stream);
int fx_finish(fx_ctx* ctx, void* stream);

/* Elapsed milliseconds of the last launch, from HIP events recorded on the launch stream
 * immediately before and after it (valid once that launch has finished). */
int fx_last_run_ms(fx_ctx* ctx, float* ms);

/* Timing marks: fx_mark records HIP event `idx` (0 <= idx < FX_MAX_MARKS) on `stream`;
 * fx_marks_ms gives the milliseconds from mark i to mark j once both have completed. */
#define FX_MAX_MARKS 256
int fx_mark(fx_ctx* ctx, int32_t idx, void* stream);
int fx_marks_ms(fx_ctx* ctx, int32_t i, int32_t j, float* ms);

/* Per-stage event timing of one iteration (the reference's MPK_EVENT_TIMING + measure.py per-op
 * gaps, docs/fleet/03-runtime.md:367-371): when iter >= 0, the next fx_run records for iteration
 * `iter` and every worker FX_PROF_SLOTS s_memrealtime stamps per stage, [stage][worker][slot]:
 * slot 0 when the worker begins the stage, slot 1 when its packet inputs have arrived, slot 2
 * when its outputs are issued, slot 3 when it leaves the stage, slots 4..7 at points inside the
 * operator (attention: scores, softmax and value product of its first tile, partials complete;
 * merge: lse weights, merged o) -- 0 where a stage has no such point.
 * fx_read_profile copies n_stages * 256 * FX_PROF_SLOTS stamps; returns the count written. */
#define FX_PROF_SLOTS 8
int fx_set_profile(fx_ctx* ctx, int32_t iter);
int fx_read_profile(fx_ctx* ctx, uint64_t* buf, int32_t n);

/* Per-iteration timestamps of the last fx_run (s_memrealtime, 100 MHz): buf[0] at the start of
 * iteration 0, buf[i] at the start of iteration i, buf[iters] at the end. Replaces the [FWD_PASS]
 * lines and event_timing.json (harness/measure.py:187-190). Returns the count written. */
int fx_read_timing(fx_ctx* ctx, uint64_t* buf, int32_t n);

/* Kernel-suite entry (kernel_tests_mi300.cu counterpart): one stage as a standalone launch of all
 * workers, with the same task split as inside fx_run; step is the decode position. Packet inputs
 * must carry tag tbase + src[k] + 1, outputs get tbase + sidx + 1; the token of an embed residual
 * is tokens(aux4)[step]. */
int fx_run_stage(fx_ctx* ctx, const fx_stage* stage, int32_t step, uint32_t tbase, int32_t sidx, void* stream);

/* Allocation-free attention (no counterpart in the reference; for callers that cannot allocate
 * device memory: code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The same work as fx_run_stage(attend) then fx_run_stage(merge) -- an MLA_ATTEND stage and its
 * MLA_MERGE_UV stage, both with or both without FX_F_MFMA -- but the split partials and the done
 * packets live in a library-owned device array (one per GPU, held until the process ends) instead
 * of the stages' partials / done buffers, which are ignored; it calls no allocating routine. The
 * attend stage runs with (tbase, sidx), the merge with (tbase, sidx + 1) and src[0] = sidx. Limit:
 * n_splits <= FX_NOALLOC_MAX_SPLITS (the array holds that many splits' partials: 5.3 MB), partials
 * rows of 516 floats; larger plans fail with FX_E_ARG. Every call on a GPU shares that GPU's array:
 * calls that overlap on one GPU race. Returns after both launches have finished. */
#define FX_NOALLOC_MAX_SPLITS 160
int fx_mla_attend_merge_noalloc(fx_ctx* ctx, const fx_stage* attend, const fx_stage* merge, int32_t step,
                                uint32_t tbase, int32_t sidx, void* stream);

/* Kernel-suite timing (the reference suite's KT_TIME, fleet/tasks/README.md:294-311): `reps` rounds
 * of standalone launches of stages[0 .. n) in turn (n copies over different weights defeat the
 * 256 MB last-level cache), back to back on `stream`; *us = mean microseconds per launch from HIP
 * events around all of them (launch gaps included). */
int fx_time_stages(fx_ctx* ctx, const fx_stage* stages, int32_t n, int32_t reps, int32_t step, uint32_t tbase,
                   int32_t sidx, void* stream, float* us);

/* ---- seeded inputs (pack_weights counterpart: fills the packed keys from a seed) -------------- */
/* dst[r * dst_stride + j] = bf16(scale * z(src_offset + r * src_stride + j)) for r < rows, j < row_len,
 * where z(i) is element i of the N(0,1) stream: Philox4x32-10 (key = seed, counter = (i / 4, stream,
 * 0x5EED)) word pairs through Box-Muller, element i % 4 of the block; bit-identical to the CPU
 * generator. A tensor is one stream; packing it (a row range, a column slice) is a strided call. */
int fx_gen_normal_bf16(fx_ctx* ctx, void* dst, uint64_t rows, uint64_t row_len, uint64_t dst_stride,
                       uint64_t src_offset, uint64_t src_stride, uint64_t seed, uint32_t stream, float scale);
int fx_fill_u16(fx_ctx* ctx, void* dst, uint64_t n, uint16_t value);

/* ---- FP8 expert weights ------------------------------------------------------------------------ */
/* Weight-only FP8 of `rows` bf16 rows of K (K % 16 == 0): dst = the rows' OCP e4m3fn codes [rows][K]
 * (w / scale rounded to nearest even, saturated at 448), then their f32 scales [rows] (max|w| / 448,
 * 1 for an all-zero row). The W13 / W2 stages read it with FX_F_FP8. The reference only projects
 * this (README.md:130 "FP8 (stretch)", docs/acceleration/04-technique-ledger.md:12, weight-only). */
int fx_quantize_fp8(fx_ctx* ctx, const void* src, void* dst, int64_t rows, int32_t K, void* stream);
/* The inverse for the batched prefill's GEMMs: dst[r][j] = bf16(e4m3(codes[r][j]) * scale[r]). */
int fx_dequantize_fp8(fx_ctx* ctx, const void* src, void* dst, int64_t rows, int32_t K, void* stream);

/* ---- batched prefill (fleet/prefill.py) ------------------------------------------------------- */
/* The prompt's forward pass over M positions at once, writing the latent-cache rows the decode
 * consumes. The reference has no prefill of its own: it captures the caches from the HF model's
 * prefill (harness/run_reference.py:367-376, 414-425; run_fleet.py:533-537 uploads them). Plain
 * GEMMs go to rocBLAS; the row work between them is this library's kernels, rounding at the
 * decode spec's points. All launches are asynchronous on `stream`. */

/* Row-major D[b] = alpha * op(A[b]) op(B[b]) + beta * C[b] for b < batch: A, B bf16, FP32 accumulate,
 * C and D bf16 (d_f32 = 0) or FP32 (d_f32 = 1); op(X) = X^T when trans_x. op(A) is [M, K] (A stored
 * [M, lda] or, transposed, [K, lda]), op(B) is [K, N] (B stored [K, ldb] or, transposed, [N, ldb]);
 * strides in elements between batch entries; C may equal D. */
int fx_gemm(fx_ctx* ctx, int32_t trans_a, int32_t trans_b, int32_t M, int32_t N, int32_t K, float alpha,
            const void* A, int64_t lda, int64_t stride_a, const void* B, int64_t ldb, int64_t stride_b, float beta,
            const void* C, int64_t ldc, int64_t stride_c, void* D, int64_t ldd, int64_t stride_d, int32_t d_f32,
            int32_t batch, void* stream);
/* x[m] = W_embed[tokens[m]] (H bf16 per row). */
int fx_pf_embed(fx_ctx* ctx, const int64_t* tokens, const void* W_embed, void* x, int32_t M, int32_t H, void* stream);
/* y[m] = rmsnorm(x[m]) * w (K bf16 per row at strides ldx / ldy elements; numpy_ref.py:54-60). */
int fx_pf_rmsnorm(fx_ctx* ctx, const void* x, int64_t ldx, const void* w, void* y, int64_t ldy, int32_t M, int32_t K,
                  float eps, void* stream);
/* MLA prep of rows m < M at positions pos0 + m (numpy_ref.py:85-103): c_kv[pos] = rmsnorm of the
 * latent, k_pe[pos] = RoPE of the rope part (both caches [s_max, .]), q_pe[m][h] = RoPE of q's rope
 * part ([M, n_heads, 64]); qkva rows [n_heads * (d_n + 64) + d_c + 64] at stride ldq. */
int fx_pf_prep(fx_ctx* ctx, const void* qkva, int64_t ldq, const void* w_kv_norm, const void* cos, const void* sin,
               void* c_kv, void* k_pe, void* q_pe, int32_t pos0, int32_t M, int32_t s_max, int32_t n_heads,
               int32_t d_n, int32_t d_c, float eps, void* stream);
/* Causal softmax of FP32 score rows i < M of `heads` heads: keys j <= key0 + i (of n_cols);
 * P = bf16(exp(S * scale - max)) (0 past the last key), l = the FP32 sum. */
int fx_pf_softmax(fx_ctx* ctx, const void* S, int64_t ldS, int64_t strideS, void* P, int64_t ldP, int64_t strideP,
                  void* l, int64_t strideL, int32_t M, int32_t heads, int32_t n_cols, int32_t key0, float scale,
                  void* stream);
/* obf[h][i][c] = bf16(O[h][i][c] / l[h][i]) (O FP32 [heads, M, d]). */
int fx_pf_attn_out(fx_ctx* ctx, const void* O, const void* l, void* obf, int32_t M, int32_t heads, int32_t d,
                   void* stream);
/* act[r][i] = bf16(silu(gu[r][i]) * gu[r][I + i]) (numpy_ref.py:248-253, 262-272). */
int fx_pf_silu(fx_ctx* ctx, const void* gu, void* act, int32_t rows, int32_t I, void* stream);
/* Router of each row (numpy_ref.py:216-227): ids [M, topk + n_shared] = top-k of softmax(logits),
 * then the shared experts E.., wts = p * scaling, then 1.0 (logits FP32 [M, E]). */
int fx_pf_route(fx_ctx* ctx, const void* logits, void* ids, void* wts, int32_t M, int32_t E, int32_t topk,
                int32_t n_shared, float scaling, void* stream);
/* dst[r] = src[idx[r]] (rows of H bf16). */
int fx_pf_gather(fx_ctx* ctx, const void* src, const void* idx, void* dst, int32_t rows, int32_t H, void* stream);
/* x_res[m] = bf16(x_mid[m] + sum_s og[inv[m][s]] * w[m][s]) in slot order (numpy_ref.py:316-321). */
int fx_pf_combine(fx_ctx* ctx, const void* x_mid, const void* og, const void* inv, const void* w, void* x_res,
                  int32_t M, int32_t H, int32_t slots, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* FLEET_MI355X_H */
