/*
 * jkv.h — C ABI of the MI355X (gfx950) hard residual-quantization hot path.
 *
 * Every entry point is `extern "C"`, takes plain device pointers, element
 * counts and strides, enqueues its work on the caller's HIP stream and never
 * synchronises the host.  The caller owns every device buffer (outputs and
 * workspaces included); the library keeps no device state between calls,
 * apart from the static scratch array of jkv_decode_attention_noalloc.
 * Return value: JKV_OK (0) or a negative JKV_E* code; jkv_last_error() then
 * returns a thread-local message.
 *
 * Layout conventions (identical to the reference operator API):
 *   states  [B,H,T,G*d]  fp16/bf16/fp32, last axis contiguous, strides in
 *                        elements for the B, H and T axes
 *   tables  [H*G,S,K,d]  fp32 masters (the kernels search and decode with
 *                        their fp16 round trip, as the reference does)
 *   codes   [B,H,T,G,S]  uint8, the (G,S) block contiguous, byte strides for
 *                        the B, H and T axes
 * Residual VQ over full head vectors is G=1, d=D; grouped CQ is S=1.
 */
#ifndef JKV_H
#define JKV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* jkv_stream_t; /* == hipStream_t */

enum {
  JKV_OK = 0,
  JKV_EINVAL = -1,   /* invalid geometry or argument            */
  JKV_EHIP = -2,     /* HIP runtime / launch error              */
  JKV_ENOTSUP = -3,  /* geometry outside what the kernels cover */
};

enum { JKV_F16 = 0, JKV_BF16 = 1, JKV_F32 = 2 };

#define JKV_MAX_EXITS 8

/* Library version (major*10000 + minor*100 + patch). */
int jkv_version(void);

/* Thread-local text of the last error raised by this thread. */
const char* jkv_last_error(void);

/* Bytes of device workspace jkv_rvq_encode needs for this geometry: the
 * whitened selector tables, or for full-vector codebooks (d = 128, K = 256,
 * S <= 32, no whitener) the fp16-deployed tables of the MFMA kernel.  Given
 * less, a full-vector call runs on the one-row-per-thread kernel instead. */
int64_t jkv_rvq_encode_workspace_bytes(int64_t H, int64_t G, int64_t S,
                                       int64_t K, int64_t d,
                                       int32_t has_whitener);

/*
 * Hard greedy residual-VQ / grouped-CQ encode with fp16-deployed codewords.
 * Replaces the stage loop of hard_residual_vq_exits
 * (src/jointkv/closed_loop_vq.py:235-410, nearest search :52-76) and the
 * search/gather of hard_grouped_cq (src/jointkv/cq_tac.py:33-114).
 *   whiteners  [H*G,d,d] fp32 or NULL: search runs in W·x coordinates with
 *              W·c tables (closed_loop_vq.py:312-330,384-390; cq_tac.py:80-85)
 *   recon[e]   [B,H,T,G*d] contiguous in the states dtype, written with
 *              fp16/bf16/fp32( sum_{s<exit_depths[e]} fp32(fp16(c_s)) )
 *              (closed_loop_vq.py:381,396-402); NULL entries are skipped.
 * Ties resolve to the lowest codeword index (torch.argmin).
 */
int jkv_rvq_encode(const void* states, int32_t states_dtype, int64_t B,
                   int64_t H, int64_t T, int64_t G, int64_t d,
                   int64_t stride_b, int64_t stride_h, int64_t stride_t,
                   const float* tables, int64_t S, int64_t K,
                   const float* whiteners, uint8_t* codes,
                   int64_t code_stride_b, int64_t code_stride_h,
                   int64_t code_stride_t, int32_t n_exits,
                   const int32_t* exit_depths, void* const* recon,
                   void* workspace, int64_t workspace_bytes,
                   jkv_stream_t stream);

/*
 * A token's K and V through jkv_rvq_encode in one call: the codec forward
 * encodes K then V with the same geometry (src/jointkv/uniform_depth_tac.py:
 * 69-101 and cq_tac.py:117-192, per decode step at
 * experiments_followup_mistral/evaluate_mistral_longbench.py:94-98).  Both
 * share B/H/T/G/d/S/K, the state strides, the code strides and the exit
 * depths; each has its own states, tables, codes and reconstructions.  With
 * fp16 states, d in {4, 8}, K = 256 and S <= 2 both run in one launch (twice
 * the workgroups of one, at the latency of one for decode-sized calls);
 * other geometries run the two encodes in turn, sharing `workspace`.  No
 * whitener (the K side's whitener needs jkv_rvq_encode).
 */
int jkv_rvq_encode_kv(const void* key_states, const void* value_states, int32_t states_dtype,
                      int64_t B, int64_t H, int64_t T, int64_t G, int64_t d, int64_t stride_b,
                      int64_t stride_h, int64_t stride_t, const float* key_tables,
                      const float* value_tables, int64_t S, int64_t K, uint8_t* key_codes,
                      uint8_t* value_codes, int64_t code_stride_b, int64_t code_stride_h,
                      int64_t code_stride_t, int32_t n_exits, const int32_t* exit_depths,
                      void* const* key_recon, void* const* value_recon, void* workspace,
                      int64_t workspace_bytes, jkv_stream_t stream);

/*
 * n_jobs encodes of one geometry in one call: a whole cache's layers and
 * their K and V, as the codec forward encodes them one layer at a time
 * (src/jointkv/uniform_depth_tac.py:69-101 called per layer).  Job j is
 * jkv_rvq_encode(states[j], ..., tables[j], ..., codes[j], ...,
 * recon + j * n_exits, ...) without a whitener; all jobs share B/H/T/G/d/S/K,
 * the state strides, the code strides and the exit depths, and each output
 * is what that call writes, bit for bit.  With fp16 states, d in {4, 8},
 * K = 256 and S <= 2, up to 64 jobs run in one launch (the first workgroups
 * of one job overlap the last of the one before, and each workgroup
 * encodes a longer row range).  Full-vector codebooks (fp16, d = 128,
 * K = 256, S <= 32, at most two exits) with
 * jkv_rvq_encode_many_workspace_bytes() of workspace run up to 64 jobs in
 * one table launch and one search launch.  Other geometries run the jobs in
 * turn, sharing `workspace`.  recon is [n_jobs][n_exits] (NULL: no
 * reconstructions).
 */
/* Bytes of workspace jkv_rvq_encode_many needs for n_jobs encodes of this
 * geometry (no whitener): for full-vector codebooks (d = 128, K = 256,
 * S <= 32) one table region per job of a launch (up to 64), so that every
 * job runs in one launch; otherwise what one jkv_rvq_encode needs. */
int64_t jkv_rvq_encode_many_workspace_bytes(int32_t n_jobs, int64_t H, int64_t G,
                                            int64_t S, int64_t K, int64_t d);

int jkv_rvq_encode_many(int32_t n_jobs, const void* const* states, int32_t states_dtype,
                        int64_t B, int64_t H, int64_t T, int64_t G, int64_t d,
                        int64_t stride_b, int64_t stride_h, int64_t stride_t,
                        const float* const* tables, int64_t S, int64_t K,
                        uint8_t* const* codes, int64_t code_stride_b,
                        int64_t code_stride_h, int64_t code_stride_t, int32_t n_exits,
                        const int32_t* exit_depths, void* const* recon, void* workspace,
                        int64_t workspace_bytes, jkv_stream_t stream);

/*
 * Codes-to-vector reconstruction with given (frozen) codes:
 * out = dtype( sum_{s<depth} fp32(fp16(tables[h*G+g, s, code])) ).
 * Replaces frozen_assignment_u16_reconstruction
 * (experiments/train_pure_uniform16_closed_loop_vq.py:395-442) and the
 * decoded workspace of LayerCache.append
 * (experiments_followup_mistral/evaluate_mistral_longbench.py:44-60).
 */
int jkv_rvq_decode(const uint8_t* codes, int64_t code_stride_b,
                   int64_t code_stride_h, int64_t code_stride_t, int64_t B,
                   int64_t H, int64_t T, int64_t G, int64_t d,
                   const float* tables, int64_t S, int64_t K, int32_t depth,
                   void* out, int32_t out_dtype, jkv_stream_t stream);

/* jkv_rvq_decode with the tables given as their fp16 deployed words
 * (fp16(masters), [H*G,S,K,d], e.g. jkv_f32_to_f16 output or a codec's
 * deployed tables): out = dtype( sum_{s<depth} fp32(tables16[h*G+g, s,
 * code]) ), the same bits as jkv_rvq_decode on the masters, reading half the
 * table bytes. */
int jkv_rvq_decode_f16(const uint8_t* codes, int64_t code_stride_b,
                       int64_t code_stride_h, int64_t code_stride_t, int64_t B,
                       int64_t H, int64_t T, int64_t G, int64_t d,
                       const void* tables16, int64_t S, int64_t K, int32_t depth,
                       void* out, int32_t out_dtype, jkv_stream_t stream);

/* Bytes of device workspace jkv_rvq_scatter_grad needs for this geometry,
 * gradient dtype and determinism request. */
int64_t jkv_rvq_scatter_workspace_bytes(int64_t B, int64_t H, int64_t T,
                                        int64_t G, int64_t d, int64_t S,
                                        int64_t K, int32_t grad_dtype,
                                        int32_t deterministic);

/*
 * Straight-through codebook gradient: for every stage s,
 *   grad_tables[h*G+g, s, k, :] += sum over rows with codes[..,g,s]==k of
 *       sum over exits e with exit_depths[e] > s of fp32(grads[e][.., g*d:(g+1)*d])
 * Replaces the autograd backward of torch.gather at
 * closed_loop_vq.py:376-381 (via the deploy STE :298) and cq_tac.py:98-99.
 * grads[e] are [B,H,T,G*d] contiguous in grad_dtype.
 * When d is a multiple of 4, a block holds the bins of one (head, group,
 * stage, slice of 8 or 4 dims) in LDS.  fp16 gradients are summed exactly in
 * 64-bit fixed point (value * 2^24) and rounded to fp32 once, so the result
 * is the correctly rounded sum and identical from run to run; bf16/fp32
 * gradients are summed with fp32 LDS atomics.  Other d, or gradient buffers
 * not aligned to the slice, use global fp32 atomics.
 * deterministic != 0 asks for a run-to-run identical result: fp16 gradients
 * already give one (and then must be aligned to the slice, else
 * JKV_EINVAL); bf16/fp32 gradients take fixed-order sums (per 256-row chunk
 * an in-order sum per codeword, then the chunk partials in chunk order).
 * May need jkv_rvq_scatter_workspace_bytes() of workspace.
 */
int jkv_rvq_scatter_grad(int32_t n_exits, const void* const* grads,
                         int32_t grad_dtype, const int32_t* exit_depths,
                         const uint8_t* codes, int64_t code_stride_b,
                         int64_t code_stride_h, int64_t code_stride_t,
                         int64_t B, int64_t H, int64_t T, int64_t G, int64_t d,
                         int64_t S, int64_t K, float* grad_tables,
                         int32_t deterministic, void* workspace,
                         int64_t workspace_bytes, jkv_stream_t stream);

/*
 * n_jobs straight-through scatters of one geometry in one call: the value
 * tables of every layer in a calibration step, whose backward runs
 * closed_loop_vq.py:376-381 once per layer.  Job j is
 * jkv_rvq_scatter_grad(n_exits, grads + j * n_exits, ..., codes[j], ...,
 * grad_tables[j], ...): all jobs share B/H/T/G/d/S/K, the code strides and
 * the exit depths.  accumulate != 0 adds into grad_tables[j] as that call
 * does; accumulate == 0 stores the sums (a fresh gradient: grad_tables[j]
 * need not be initialised, and codewords no row picks get 0).  fp16
 * gradients with one exit, aligned to the 8- (or 4-) element slice, run up
 * to 64 jobs per launch on the exact fixed-point bins over every row (one
 * block per job, head and group taking all stages when d = 8, else per
 * stage and slice), bit-identical to the one-job call; other jobs run one call each, sharing `workspace` (sized by
 * jkv_rvq_scatter_workspace_bytes for one job).
 */
int jkv_rvq_scatter_grad_many(int32_t n_jobs, int32_t n_exits, const void* const* grads,
                              int32_t grad_dtype, const int32_t* exit_depths,
                              const uint8_t* const* codes, int64_t code_stride_b,
                              int64_t code_stride_h, int64_t code_stride_t, int64_t B,
                              int64_t H, int64_t T, int64_t G, int64_t d, int64_t S,
                              int64_t K, float* const* grad_tables, int32_t accumulate,
                              int32_t deterministic, void* workspace,
                              int64_t workspace_bytes, jkv_stream_t stream);

/*
 * Squared L2 norm of each of n fp32 buffers, accumulated in fp64, written to
 * out_sumsq[n] (device).  Replaces the per-table torch.linalg.vector_norm of
 * clip_codebook_gradients
 * (experiments/train_pure_uniform16_closed_loop_vq.py:1151-1304).
 */
int jkv_sumsq(int32_t n, const float* const* buffers, const int64_t* numels,
              double* out_sumsq, jkv_stream_t stream);

/*
 * In-place grad[i] *= scales[i] (the clip_grad_norm_ multiply) and, when
 * lr != 0, the plain SGD update param[i] -= lr * grad[i]
 * (train_mistral_v_only.py:128,153: SGD, no momentum, no weight decay).
 * params may be NULL when lr == 0.  scales is a host array.
 */
int jkv_scale_sgd(int32_t n, float* const* params, float* const* grads,
                  const int64_t* numels, const float* scales, float lr,
                  jkv_stream_t stream);

/*
 * Fused decode attention over a packed uint8 code cache (one new query token
 * per sequence).  Replaces the decode branch of attention_forward
 * (evaluate_mistral_longbench.py:112-122): decoded K̂/V̂ window
 * (LayerCache.visible :62-70), RoPE of q at its position and of K̂ at the
 * absolute key positions (:114-118), repeat_kv (:119-120) and SDPA without
 * mask (:121-122), in one pass that never writes K̂ or V̂.
 *   q        [B,QH,D] fp16 (pre-RoPE), row stride q_stride_b / q_stride_h
 *   k_codes, v_codes  [B,KVH,cap,G,S] uint8 (byte strides b, h; token
 *            stride G*S); key position p lives in slot p % cap
 *   k_tables, v_tables  fp16 deployed codebooks [KVH*G,S,K,d]; K = 256,
 *            G*d = 128 with d in {4, 8} (S <= 8) or d = 128, G = 1
 *            (full-vector codebooks, S <= 32)
 *   lengths  [B] int32 device: tokens in the cache including the new one;
 *            query position = lengths[b]-1; visible keys are the last
 *            min(window, lengths[b]) positions
 *   rope_table  jkv_rope_table() output covering positions [0, rope_len),
 *            rope_len > max(lengths) - 1
 *   out      [B,QH,D] fp16 contiguous
 *   workspace  jkv_decode_workspace_bytes() bytes (split-KV partials)
 */
int64_t jkv_decode_workspace_bytes(int64_t B, int64_t QH, int64_t D,
                                   int64_t window);
int jkv_decode_attention(const void* q, int64_t q_stride_b,
                         int64_t q_stride_h, const uint8_t* k_codes,
                         const uint8_t* v_codes, int64_t code_stride_b,
                         int64_t code_stride_h, int64_t cap,
                         const void* k_tables, const void* v_tables, int64_t B,
                         int64_t QH, int64_t KVH, int64_t G, int64_t d,
                         int64_t S, int64_t K, const int32_t* lengths,
                         int64_t window, const void* rope_table,
                         int64_t rope_len, void* out, void* workspace,
                         int64_t workspace_bytes, jkv_stream_t stream);

/*
 * One decode step with the new token's append fused in: the greedy residual
 * codes of the raw K and V of the token at position lengths[b]-1 (the
 * codec call and LayerCache.append of evaluate_mistral_longbench.py:94-98)
 * are computed inside the attention launch from the tables it stages
 * anyway, written to slot (lengths[b]-1) % cap of k_codes / v_codes, and
 * attended over with the rest of the window (:112-122).
 *   k_new, v_new  [B,KVH,128] fp16 raw (pre-RoPE) head vectors, element
 *            strides new_stride_b / new_stride_h, rows 16-byte aligned
 *   the codes: fp16(tables) searched stage by stage on the fp32 residual,
 *            lowest index on ties; codes equal the reference's wherever its
 *            best/second-best margin is clear (the same rule as
 *            jkv_rvq_encode); rows with lengths[b] = 0 append nothing
 * Other arguments as jkv_decode_attention.  Serves d = 8, G = 16, S in
 * {1, 2}, K = 256 with 16-byte aligned codes and tables (the GSRQ-1/2 and
 * grouped-CQ caches); other geometries return JKV_ENOTSUP (encode with
 * jkv_rvq_encode_kv, then call jkv_decode_attention).
 */
int jkv_decode_attention_append(const void* q, int64_t q_stride_b,
                                int64_t q_stride_h, const void* k_new,
                                const void* v_new, int64_t new_stride_b,
                                int64_t new_stride_h, uint8_t* k_codes,
                                uint8_t* v_codes, int64_t code_stride_b,
                                int64_t code_stride_h, int64_t cap,
                                const void* k_tables, const void* v_tables,
                                int64_t B, int64_t QH, int64_t KVH, int64_t G,
                                int64_t d, int64_t S, int64_t K,
                                const int32_t* lengths, int64_t window,
                                const void* rope_table, int64_t rope_len,
                                void* out, void* workspace,
                                int64_t workspace_bytes, jkv_stream_t stream);

/*
 * Allocation-free variant of jkv_decode_attention.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments, results and errors as jkv_decode_attention without the
 * workspace: the split partials go to a file-scope device array of the
 * library (one per GPU, jkv_decode_noalloc_max_workspace_bytes() = 16 MiB,
 * held until the process ends).  Calls whose kernel needs more partial
 * space than that return JKV_EINVAL: B*QH*n_splits*(128+2)*4 bytes, with
 * n_splits = ceil(window/2048) for group dims 4 and 8 on 16-byte aligned
 * codes and tables (e.g. config 4 up to B*QH = 16,131 at a 4096-token
 * window) and ceil(window/256) otherwise (the bound that
 * jkv_decode_workspace_bytes reports).  The array is looked up on the first call on each
 * device (the current HIP device); no call allocates or frees memory.  Every
 * call on a device shares that device's array: calls that overlap on one
 * GPU (two streams, two threads) race and must be serialised by the caller.
 */
int64_t jkv_decode_noalloc_max_workspace_bytes(void);
int jkv_decode_attention_noalloc(const void* q, int64_t q_stride_b,
                                 int64_t q_stride_h, const uint8_t* k_codes,
                                 const uint8_t* v_codes, int64_t code_stride_b,
                                 int64_t code_stride_h, int64_t cap,
                                 const void* k_tables, const void* v_tables,
                                 int64_t B, int64_t QH, int64_t KVH, int64_t G,
                                 int64_t d, int64_t S, int64_t K,
                                 const int32_t* lengths, int64_t window,
                                 const void* rope_table, int64_t rope_len,
                                 void* out, jkv_stream_t stream);

/*
 * Decode attention over a decoded fp16 K̂/V̂ window, the reference's own
 * decode path (evaluate_mistral_longbench.py:112-122 over LayerCache's
 * decoded_key/decoded_value, :44-70), for codecs whose codewords do not fit
 * the packed-code kernel's LDS (full-vector R16/R32 tables).  Same rotary,
 * GQA, window and output as jkv_decode_attention.
 *   k_window, v_window  [B,KVH,cap,128] fp16, rows contiguous and 16-byte
 *            aligned; element strides kv_stride_b / kv_stride_h; key
 *            position p lives in slot p % cap
 *   workspace  jkv_decode_workspace_bytes(B, QH, 128, window) bytes
 */
int jkv_decode_attention_window(const void* q, int64_t q_stride_b,
                                int64_t q_stride_h, const void* k_window,
                                const void* v_window, int64_t kv_stride_b,
                                int64_t kv_stride_h, int64_t cap, int64_t B,
                                int64_t QH, int64_t KVH, const int32_t* lengths,
                                int64_t window, const void* rope_table,
                                int64_t rope_len, void* out, void* workspace,
                                int64_t workspace_bytes, jkv_stream_t stream);

/*
 * Causal sliding-window GQA prefill attention over one chunk's quantized K̂/V̂.
 * Replaces the prefill branch of attention_forward
 * (experiments_followup_mistral/evaluate_mistral_longbench.py:101-111) and its
 * training twin (experiments/train_full_model_closed_loop_vq.py:277-304):
 * RoPE of q and K̂ at positions start_positions[b] + t (the reference's fp16
 * rotary arithmetic), repeat_kv, and SDPA where query t sees keys s with
 * s <= t and t - s < window (the model's causal + sliding-window mask).
 *   q        [B,QH,T,128] fp16 pre-RoPE, element strides (b, h, t)
 *   k, v     [B,KVH,T,128] fp16 pre-RoPE chunk K̂/V̂ (e.g. encode exits or
 *            jkv_rvq_decode output), element strides (b, h, t)
 *   start_positions  [B] int32 device
 *   rope_table  jkv_rope_table() output, rope_len > max position
 *   out      [B,QH,T,128] fp16 contiguous
 *   lse      [B,QH,T] fp32 contiguous or NULL: each row's log-sum-exp of
 *            its visible scores q.k/sqrt(128) (natural log), what the
 *            backward jkv_prefill_attention_value_grad recomputes P from
 * Strides must be multiples of 8 elements and buffers 16-byte aligned.
 */
int jkv_prefill_attention(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                          int64_t q_stride_t, const void* k,
                          int64_t k_stride_b, int64_t k_stride_h,
                          int64_t k_stride_t, const void* v,
                          int64_t v_stride_b, int64_t v_stride_h,
                          int64_t v_stride_t, int64_t B, int64_t QH,
                          int64_t KVH, int64_t T, int64_t D,
                          const int32_t* start_positions, int64_t window,
                          const void* rope_table, int64_t rope_len, void* out,
                          float* lse, jkv_stream_t stream);

/*
 * jkv_prefill_attention over a chunk given as codes: the same attention, with
 * each K̂/V̂ tile rebuilt from uint8 codes while it loads (16-byte codeword
 * gathers from the fp16 deployed tables, fp16 of the fp32 stage sum), so K̂
 * and V̂ are never written to memory.  Replaces the decode-then-attend of the
 * quantized prefill branch (experiments_followup_mistral/
 * evaluate_mistral_longbench.py:101-111 with the codec's reconstruction of
 * src/jointkv/closed_loop_vq.py:298-300); output and lse are bit-identical
 * to jkv_rvq_decode at depth S followed by jkv_prefill_attention.
 *   q        as for jkv_prefill_attention
 *   k_codes, v_codes  uint8 [B,KVH,T,G,S] with byte strides (b, h, t) shared
 *            by both, the (G,S) block contiguous; even strides and addresses
 *   k_tables, v_tables  fp16 deployed tables [KVH*G][S][K][d] contiguous
 *   G, d, S, K  16, 8, 1 or 2, 256 (other geometries: JKV_ENOTSUP, for the
 *            jkv_rvq_decode + jkv_prefill_attention path)
 *   start_positions, window, rope_table, rope_len, out, lse  as for
 *            jkv_prefill_attention
 */
int jkv_prefill_attention_codes(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                int64_t q_stride_t, const uint8_t* k_codes, const uint8_t* v_codes,
                                int64_t code_stride_b, int64_t code_stride_h, int64_t code_stride_t,
                                const void* k_tables, const void* v_tables, int64_t B, int64_t QH,
                                int64_t KVH, int64_t T, int64_t G, int64_t d, int64_t S, int64_t K,
                                const int32_t* start_positions, int64_t window,
                                const void* rope_table, int64_t rope_len, void* out, float* lse,
                                jkv_stream_t stream);

/*
 * Value gradient of jkv_prefill_attention: for every key s of the chunk,
 *   d_value[b,kvh,s,:] = sum over the kv head's query heads h and rows t of
 *                        P[b,h,t,s] * d_out[b,h,t,:]
 * with P = exp(RoPE(q).RoPE(K̂) / sqrt(128) - lse[b,h,t]) under the same
 * causal sliding-window mask.  The value leg of the SDPA backward that the
 * reference's V-only calibration step runs (loss.backward() through the
 * closed-loop attention of experiments/train_full_model_closed_loop_vq.py:
 * 277-304, step at experiments_followup_mistral/train_mistral_v_only.py:
 * 142-150); K tables and backbone are frozen there, so no query or key
 * gradient is formed.
 *   q, k     as for jkv_prefill_attention (pre-RoPE fp16)
 *   d_out    [B,QH,T,128] fp16 gradient of the attention output
 *   lse      [B,QH,T] fp32 from jkv_prefill_attention
 *   d_value  [B,KVH,T,128] fp32 contiguous (written, not accumulated)
 *   workspace  jkv_prefill_value_grad_workspace_bytes() bytes, 16-byte
 *            aligned: the rotated queries [B,QH,T,128] fp16, and when a key
 *            block's query rows are split into runs that fill the device
 *            evenly, the runs' partial slots that a second kernel adds up
 * Deterministic: each key's sum runs over the heads, rows and runs in one
 * fixed order.  Limits (JKV_EINVAL past them): B and QH < 65536, T < 2^30,
 * rope_len < 2^23, and for the query heads of one kv head under 2^31 bytes
 * of rotated queries (QH/KVH * T * 256), of d_out ((QH/KVH - 1) * stride_h
 * + (T - 1) * stride_t + 128 elements) and of lse.
 */
int jkv_prefill_attention_value_grad(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                     int64_t q_stride_t, const void* k, int64_t k_stride_b,
                                     int64_t k_stride_h, int64_t k_stride_t, const void* d_out,
                                     int64_t d_stride_b, int64_t d_stride_h, int64_t d_stride_t,
                                     const float* lse, int64_t B, int64_t QH, int64_t KVH, int64_t T,
                                     int64_t D, const int32_t* start_positions, int64_t window,
                                     const void* rope_table, int64_t rope_len, float* d_value,
                                     void* workspace, int64_t workspace_bytes, jkv_stream_t stream);

/* Workspace of jkv_prefill_attention_value_grad for this geometry (bytes):
 * the runs' partial slots when there are several, then the rotated queries. */
int64_t jkv_prefill_value_grad_workspace_bytes(int64_t B, int64_t QH, int64_t KVH, int64_t T, int64_t window);

/*
 * The full backward of jkv_prefill_attention (the SDPA backward under the
 * reference's loss.backward() through its closed-loop attention,
 * experiments/train_full_model_closed_loop_vq.py:277-304), for the gradients
 * that are not NULL:
 *   d_query [B,QH,T,128], d_key [B,KVH,T,128], d_value [B,KVH,T,128], fp32
 *   contiguous, with respect to the PRE-RoPE q and K̂ (the rotary's transpose
 *   is applied) and V̂; the key and value gradients are summed over the GQA
 *   group.
 * dS = P (dO V̂ᵀ - rowsum(dO * O)), dQ = dS K̂ / sqrt(128), dK = dSᵀ Q /
 * sqrt(128), dV = Pᵀ dO, with P recomputed from the forward's lse.
 *   out      the forward output [B,QH,T,128] fp16 (for rowsum(dO * O))
 *   workspace  jkv_prefill_backward_workspace_bytes() bytes, 16-byte aligned
 * Query heads per kv head: 1, 2 or a multiple of 4.  Deterministic.  The
 * value leg has the limits of jkv_prefill_attention_value_grad.
 */
int jkv_prefill_attention_backward(const void* q, int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_t,
                                   const void* k, int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_t,
                                   const void* v, int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_t,
                                   const void* out, int64_t o_stride_b, int64_t o_stride_h, int64_t o_stride_t,
                                   const void* d_out, int64_t d_stride_b, int64_t d_stride_h,
                                   int64_t d_stride_t, const float* lse, int64_t B, int64_t QH, int64_t KVH,
                                   int64_t T, int64_t D, const int32_t* start_positions, int64_t window,
                                   const void* rope_table, int64_t rope_len, float* d_query, float* d_key,
                                   float* d_value, void* workspace, int64_t workspace_bytes,
                                   jkv_stream_t stream);

/* Workspace of jkv_prefill_attention_backward (bytes). */
int64_t jkv_prefill_backward_workspace_bytes(int64_t B, int64_t QH, int64_t KVH, int64_t T, int64_t window);

/*
 * The key-gradient leg of jkv_prefill_attention_backward alone, given
 * delta = rowsum(dO * O) [B,QH,T] fp32 (the backward computes it in its query
 * leg).  Same buffers and workspace rule as jkv_prefill_attention_value_grad
 * (which sizes it for the rotated queries too; this leg needs only the
 * slots).
 */
int jkv_prefill_attention_key_grad(const void* q, int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_t,
                                   const void* k, int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_t,
                                   const void* v, int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_t,
                                   const void* d_out, int64_t d_stride_b, int64_t d_stride_h,
                                   int64_t d_stride_t, const float* lse, const float* delta, int64_t B,
                                   int64_t QH, int64_t KVH, int64_t T, int64_t D,
                                   const int32_t* start_positions, int64_t window, const void* rope_table,
                                   int64_t rope_len, float* d_key, void* workspace, int64_t workspace_bytes,
                                   jkv_stream_t stream);

/* fp32 nearest codeword of every row: states [H,N,D] and tables [H,K,D]
 * contiguous fp32 (not deployed to fp16), D in 1..128, N below 2^30 rows
 * per head (one 256-thread block per 64 rows; larger N returns JKV_EINVAL);
 * indices [H,N] int64 receive argmin_k (|x|^2 + |c_k|^2) - 2 x.c_k, the
 * lowest k on ties.
 * Replaces `_nearest_indices` without whiteners
 * (src/jointkv/nested_vq.py:178-215), the search of the offline multi-exit
 * additive coordinate refinement (nested_vq.py:583-741).
 */
int jkv_nearest_f32(const float* states, int64_t H, int64_t N, int64_t D,
                    const float* tables, int64_t K, int64_t* indices,
                    jkv_stream_t stream);

/* The M (1..8, M < K) nearest fp32 codewords of every row, nearest first
 * (equal distances in index order): states [H,N,D], tables [H,K,D] as for
 * jkv_nearest_f32; excluded [H,N] int64 or NULL, one index per row left out
 * of the search; indices [H,N,M] int64.  Replaces `_nearest_topk_indices`
 * (src/jointkv/nested_vq.py:218-260), the shortlist search of the offline
 * multi-exit additive block refinement (nested_vq.py:757-1001).
 */
int jkv_nearest_topk_f32(const float* states, int64_t H, int64_t N, int64_t D,
                         const float* tables, int64_t K, int64_t M,
                         const int64_t* excluded, int64_t* indices,
                         jkv_stream_t stream);

/*
 * One sliding-pair step of the offline multi-exit additive block refinement:
 * replaces the Cartesian scoring and update of one (stage, stage+1) block of
 * `multi_exit_additive_block_refinement` (src/jointkv/nested_vq.py:838-958).
 *   states     [H][N][D] fp32 rows x
 *   recon      [n_recon][H][N][D] fp32 reconstruction of each exit, updated
 *              in place for the n_exits exits listed
 *   exit_slots, exit_weights, exit_has_second  (host arrays, n_exits <= 32):
 *              the weighted exits that contain the first stage, their
 *              weight and whether they also contain the second stage
 *   first_table [H][K1][D], second_table [H][K2][D] fp32 codebooks
 *   first_shortlist, second_shortlist  [H][N][L] int64 (1 <= L <= 9): entry
 *              0 is the current index, the rest its alternatives, each in
 *              [0, K)
 *   first_out, second_out  [H][N] int64: the chosen indices
 * The pair (i, j) minimises sum_m w_m |(x - r_m) + c1[cur1] + s_m c2[cur2]
 * - c1[i] - s_m c2[j]|^2 (s_m = exit m contains the second stage), the
 * lowest i*L + j (the current pair first) on equal cost; each listed
 * reconstruction then moves by the chosen words' changes, first stage first.
 */
int jkv_pair_block_select(const float* states, float* recon, int64_t n_recon,
                          int64_t H, int64_t N, int64_t D, int32_t n_exits,
                          const int32_t* exit_slots, const float* exit_weights,
                          const int32_t* exit_has_second,
                          const float* first_table, const float* second_table,
                          int64_t K1, int64_t K2,
                          const int64_t* first_shortlist,
                          const int64_t* second_shortlist, int64_t L,
                          int64_t* first_out, int64_t* second_out,
                          jkv_stream_t stream);

/*
 * Per-codeword sums of one k-means update of the offline gain-shape parent
 * fitting: replaces the index_add_ calls of `fit_residual_stages`
 * (experiments/build_frozen_gsrq_multi_exit.py:547-606).  For every head h
 * and codeword k, over the rows n with indices[h,n] = k, in row order:
 *   raw_sums[h,k,:]     = sum w[h,n] * x[h,n,:]
 *   shape_sums[h,k,:]   = sum (x[h,n,:] / max(|x[h,n,:]|, 1e-8)) * w[h,n]
 *                         (only when with_shapes)
 *   denominators[h,k]   = sum w[h,n]
 * with w = 1 when weights is NULL (the products are then skipped, so the
 * raw sums are the plain row sums).
 *   rows [H,N,D] fp32 (D in 1..128), indices [H,N] int64, weights [H,N] fp32
 *   or NULL; outputs [H,K,D], [H,K,D], [H,K] fp32 contiguous (overwritten).
 *   workspace  jkv_gain_shape_sums_workspace_bytes() bytes (may be NULL when
 *            that is 0): row slices write partial sums that a second kernel
 *            adds in slice order, so the sums do not depend on scheduling.
 * Rows whose index lies outside [0, K) are skipped.
 */
int jkv_gain_shape_sums(const float* rows, int64_t H, int64_t N, int64_t D,
                        const int64_t* indices, const float* weights, int64_t K,
                        int32_t with_shapes, float* shape_sums, float* raw_sums,
                        float* denominators, void* workspace,
                        int64_t workspace_bytes, jkv_stream_t stream);

/* Workspace of jkv_gain_shape_sums for this geometry (bytes). */
int64_t jkv_gain_shape_sums_workspace_bytes(int64_t H, int64_t N, int64_t D,
                                            int64_t K, int32_t with_shapes);

/*
 * residual[h,n,:] -= tables[h, indices[h,n], :] in place (fp32; residual
 * [H,N,D], tables [H,K,D], indices [H,N] int64; rows with an index outside
 * [0, K) are left unchanged): the per-stage residual update of
 * `fit_residual_stages` (build_frozen_gsrq_multi_exit.py:617-628).
 */
int jkv_subtract_codewords(float* residual, int64_t H, int64_t N, int64_t D,
                           const float* tables, int64_t K,
                           const int64_t* indices, jkv_stream_t stream);

/*
 * Rotary table for head_dim 128, fp16 [n_pos][2][64] (per position the cos of
 * the 64 frequencies, then their sin):
 * angle = fp32(p) * inv_freq[i] in fp32, cos/sin in fp32 rounded to fp16 —
 * the arithmetic of the reference's rotary module
 * (transformers' MistralRotaryEmbedding behind
 * experiments_followup_mistral/evaluate_mistral_longbench.py:102,113,117).
 * inv_freq: 64 fp32 device values (computed on the host the same way).
 */
int jkv_rope_table(const float* inv_freq, int64_t n_pos, void* out,
                   jkv_stream_t stream);

/* fp32 -> fp16 copy (the deploy round trip tables.half()), n elements. */
int jkv_f32_to_f16(const float* src, void* dst, int64_t n, jkv_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* JKV_H */
