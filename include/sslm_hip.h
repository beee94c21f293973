/* sslm_hip.h -- the C ABI of the MI355X (gfx950) backend of SuperSLM's integer forward path.
 *
 * Drop-in boundary: libsslm_hip.so exports the reference's own sslm_* verbs with the reference's
 * signatures, handle types, struct layouts and status codes, so a host that links the reference
 * library (include/superslm/sslm_abi.h + sslm_abi_functions*.inc) relinks against this one
 * unchanged.  Each declaration names the reference declaration it replaces.  Plain pointers and
 * sizes only; no torch or HIP types cross this boundary.
 *
 * Residency: the model's weights, every KV block and every sequence's stream state live in HBM.
 * The caller-owned KV-pool and workspace buffers are still required and validated exactly as the
 * reference validates them (size, 64-byte alignment) and hold only host bookkeeping.
 *
 * Verbs outside the integer forward path (tokenizer, prefixes, detokenize) are exported with
 * their reference signatures and return SSLM_INVALID_ARGUMENT.
 */
#ifndef SSLM_HIP_H
#define SSLM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* opaque handles -- reference include/superslm/sslm_abi.h:11-27 */
typedef struct sslm_model_s* sslm_model;
typedef struct sslm_seq_s* sslm_seq;
typedef struct sslm_prefix_s* sslm_prefix;
typedef struct sslm_adapter_s* sslm_adapter;
typedef struct sslm_kv_pool_s* sslm_kv_pool;
typedef struct sslm_workspace_s* sslm_workspace;
typedef struct sslm_schema_s* sslm_schema;

/* reference sslm_abi.h:40-46 */
typedef struct sslm_config {
	int32_t max_batch;
	int32_t max_chunk_budget;
	int32_t max_layer_budget;
	uint32_t reserved;
} sslm_config;

/* reference sslm_abi.h:57-61 */
typedef struct sslm_detok_state {
	uint8_t pending_bytes[3];
	uint8_t pending_count;
} sslm_detok_state;

/* reference sslm_abi.h:96-152 (same values, same order) */
typedef enum sslm_status {
	SSLM_OK = 0,
	SSLM_INVALID_ARGUMENT,
	SSLM_BUFFER_TOO_SMALL,
	SSLM_MISALIGNED_BUFFER,
	SSLM_ARTIFACT_REJECTED,
	SSLM_ADAPTER_MODEL_MISMATCH,
	SSLM_RESTORE_MODEL_MISMATCH,
	SSLM_RESTORE_KV_MISMATCH,
	SSLM_MODEL_HAS_LIVE_SEQUENCES,
	SSLM_POOL_HAS_LIVE_HANDLES,
	SSLM_ADAPTER_HAS_LIVE_SEQUENCES,
	SSLM_ADAPTER_SWAP_MIDTOKEN_REJECTED,
	SSLM_SEQ_RESET_MIDTOKEN_REJECTED,
	SSLM_PREFIX_FROZEN_REJECTED,
	SSLM_KV_POOL_EXHAUSTED,
	SSLM_TOKEN_ID_OUT_OF_RANGE,
	SSLM_CONTEXT_CAP_EXCEEDED,
	SSLM_TOKEN_ID_UNMAPPED,
	SSLM_SCHEMA_NOT_FOUND,
	SSLM_SCHEMA_BIND_REJECTED,
	SSLM_SCHEMA_SPAN_UNBOUND,
	SSLM_PREFIX_SCHEMA_MISMATCH,
	SSLM_RESTORE_SCHEMA_MISMATCH,
	SSLM_SCHEMA_SPAN_UNREACHABLE,
	SSLM_SCHEMA_UNSATISFIABLE,
	SSLM_ALLOCATION_FAILED,
	SSLM_NUMERIC_STEP_REFUSED,
	SSLM_STATUS_NEXT_FREE
} sslm_status;

/* reference sslm_abi.h:160-163 */
typedef enum sslm_span_kind { SSLM_SPAN_PROMPT = 0, SSLM_SPAN_SCHEMA_CONTENT = 1 } sslm_span_kind;

#define SSLM_DECODE_MODE_GREEDY 0
#define SSLM_DECODE_MODE_DAMPED_GREEDY 1
/* reference sslm_abi.h:194-196: sslm_decode_params_init's damped-greedy defaults */
#define SSLM_DAMPED_GREEDY_DEFAULT_ALPHA_Q15 65536
#define SSLM_DAMPED_GREEDY_DEFAULT_ANTI_LM_ORDER 2
#define SSLM_DAMPED_GREEDY_DEFAULT_TOP_K 6

/* reference sslm_abi.h:207-224 */
typedef struct sslm_decode_params {
	int32_t layer_budget;
	uint32_t struct_size;
	int32_t mode;
	int32_t alpha_q15;
	int32_t anti_lm_max_order;
	int32_t top_k;
	int64_t q_ln2;
	int64_t q_b;
	int64_t q_c;
} sslm_decode_params;

/* reference sslm_abi.h:232-238 */
typedef struct sslm_stats_out {
	int64_t decode_step_ceiling;
	int64_t decode_step_actual;
	int64_t forced_token_count;
	int32_t kv_blocks_resident;
	int32_t schema_accepting;
} sslm_stats_out;

#define SSLM_ABI_ALIGNMENT_BYTES 64u

/* ---- model ---- reference sslm_abi_functions_g5_comparable.inc (line of each verb) */
sslm_status sslm_model_map(const void* data, size_t size, sslm_model* out);          /* :23 */
sslm_status sslm_model_unmap(sslm_model model);                                      /* :24 */
size_t sslm_kv_block_size(sslm_model model);                                         /* :25 */
size_t sslm_kv_pool_overhead_size(sslm_model model, uint32_t block_count);           /* :26 */
size_t sslm_seq_state_size(sslm_model model);                                        /* :27 */
sslm_status sslm_kv_pool_create(sslm_model model, void* buf, size_t buf_size, uint32_t block_count,
                                sslm_kv_pool* out);                                  /* :28 */
sslm_status sslm_kv_pool_destroy(sslm_kv_pool pool);                                 /* :30 */
sslm_status sslm_workspace_destroy(sslm_workspace ws);                               /* :31 */

/* ---- sequences ---- */
sslm_status sslm_seq_create(sslm_model model, sslm_kv_pool* pool, sslm_seq* out);    /* :38 */
sslm_status sslm_seq_release(sslm_seq seq);                                          /* :39 */
sslm_status sslm_seq_reset(sslm_seq seq);                                            /* :40 */
/* SSB3 sequence blob, byte-identical to the reference's (src/sslm_abi.cpp:2585-2720); the
 * two-call sizing form (buf NULL) sets *n and returns SSLM_BUFFER_TOO_SMALL */
sslm_status sslm_seq_save(sslm_seq seq, void* buf, size_t* n);                       /* :42 */
/* SSB3 or SSB2 blob into a block of `pool`, checked in the reference's order
 * (src/sslm_abi.cpp:2722-2987) */
sslm_status sslm_seq_restore(sslm_model model, sslm_kv_pool* pool, const void* buf, size_t n,
                             sslm_seq* out);                                         /* :43 */
sslm_status sslm_seq_set_adapter(sslm_seq seq, sslm_adapter adapter);                /* :45 */
sslm_status sslm_adapter_map(const void* data, size_t size, sslm_model base, sslm_adapter* out); /* :46 */
sslm_status sslm_adapter_release(sslm_adapter adapter);                              /* :47 */
size_t sslm_adapter_residency(sslm_adapter adapter);                                 /* :48 */

/* ---- SCM1 schemas (src/sslm_abi.cpp:1236-1264, 1791-1818) ---- */
sslm_status sslm_schema_lookup(sslm_model model, const char* name, sslm_schema* out);
size_t sslm_schema_count(sslm_model model);
sslm_status sslm_schema_name(sslm_model model, int32_t index, char* buf, size_t* n);
sslm_status sslm_seq_set_schema(sslm_seq seq, sslm_schema schema);

/* ---- the hot path ---- */
sslm_status sslm_prefill(sslm_model model, sslm_seq seq, const int32_t* tokens, int32_t count,
                         int32_t chunk_budget, sslm_span_kind kind, sslm_workspace ws,
                         int32_t* consumed);                                         /* :49 */
sslm_status sslm_decode_step(sslm_model model, sslm_seq* seqs, int32_t n, const sslm_decode_params* params,
                             sslm_workspace ws, int32_t* out_tokens);                /* :52 */
sslm_status sslm_stats(sslm_model model, sslm_seq seq, sslm_stats_out* out);         /* :56 */

/* reference sslm_abi_functions.inc:23-52 */
sslm_status sslm_decode_step_v2(sslm_model model, sslm_seq* seqs, int32_t n, const sslm_decode_params* params,
                                sslm_workspace ws, int32_t* out_tokens);
sslm_status sslm_decode_params_init(sslm_model model, int32_t mode, int32_t layer_budget, sslm_decode_params* out);
size_t sslm_workspace_size(sslm_model model, const sslm_config* config);
sslm_status sslm_workspace_create(sslm_model model, const sslm_config* config, void* buf, size_t buf_size,
                                  sslm_workspace* out);

/* reference src/sslm_abi.cpp:3366 -- test seam: one KV block's bytes in the reference layout
 * [layer][K|V][kv_head][context_cap][head_dim], read back from HBM. */
sslm_status sslm_g5_test_only_peek_kv_block_bytes(sslm_kv_pool pool, uint32_t block_index, uint8_t* out_buf,
                                                  size_t n);

/* ---- outside the integer forward path: exported, always SSLM_INVALID_ARGUMENT ---- */
sslm_status sslm_prefix_begin(sslm_model model, sslm_kv_pool* pool, sslm_prefix* out);
sslm_status sslm_prefix_prefill(sslm_model model, sslm_prefix prefix, const int32_t* tokens, int32_t count,
                                int32_t chunk_budget, sslm_span_kind kind, sslm_workspace ws, int32_t* consumed);
sslm_status sslm_prefix_freeze(sslm_prefix prefix);
sslm_status sslm_prefix_release(sslm_prefix prefix);
sslm_status sslm_seq_adopt_prefix(sslm_seq seq, sslm_prefix prefix);
sslm_status sslm_tokenize(sslm_model model, const char* utf8, int32_t* tokens, int32_t* n);
sslm_status sslm_prefix_set_schema(sslm_prefix prefix, sslm_schema schema);
sslm_status sslm_detokenize_stream(sslm_model model, sslm_detok_state* state, const int32_t* tokens, int32_t n,
                                   char* utf8, int32_t* out_n);

/* ---- backend extras (no reference counterpart) ---- */

/* Kernel-class timing, for benchmarks: when enabled, every launch of the hot path is bracketed
 * with HIP events on the library's stream and accumulated per class.  Classes: 0 projection
 * GEMM/GEMV, 1 LM-head GEMV, 2 attention, 3 row kernels (norm/funnel/residual/act/landing),
 * 4 LoRA.  `bytes` is the algorithmic weight+activation traffic of the GEMM classes. */
#define SSLM_HIP_PROFILE_CLASSES 5
void sslm_hip_profile_enable(int on);
void sslm_hip_profile_read(double* ms, int64_t* launches, int64_t* bytes, int64_t* ops, int classes);
void sslm_hip_profile_reset(void);
/* The decode GEMVs of one step for M tokens -- every layer's q|k|v, o, gate|up and down
 * projections with that layer's own weights, in the layer loop's order, then the LM head --
 * launched back to back `iters` times between two HIP events on the model's stream (so every
 * weight byte streams from HBM, as in a step).  Writes us[0] = mean microseconds per pass,
 * bytes[0] = algorithmic bytes per pass (weights + activations + outputs + fold tables) and
 * shapes[0] = launches per pass; with cap >= 6 also, per projection class c = 1..5 (q|k|v, o,
 * gate|up, down, LM head), the same for a pass of that class's launches alone (all layers').
 * Returns 1, or -1.  Sequence state is not touched. */
int32_t sslm_hip_bench_decode_gemv(sslm_model model, int32_t M, int32_t iters, double* us, int64_t* bytes,
                                   int64_t* shapes, int32_t cap);
/* The same passes as sslm_hip_bench_decode_gemv with every GEMV replaced by a plain streaming
 * read of its weight buffer (the packed decode copy where there is one): the HBM rate a launch
 * sequence of that shape -- the same launches, bytes and order -- reaches at all.  bytes[] count
 * the weight bytes read.  No counterpart in the reference; a bench reference point. */
int32_t sslm_hip_bench_read_floor(sslm_model model, int32_t M, int32_t iters, double* us, int64_t* bytes,
                                  int64_t* shapes, int32_t cap);
/* The projection GEMMs of one M-token prefill chunk (65 <= M <= 512) -- every layer's q|k|v, o,
 * gate|up and down, each layer's own weights, the layer loop's launch shapes -- back to back
 * `iters` times between two HIP events on the model's stream.  Writes us[0] = mean
 * microseconds per pass, ops[0] = 2*M*N*K summed over the pass, launches[0] = launches per
 * pass; returns 1, or -1.  Sequence state is not touched. */
int32_t sslm_hip_bench_prefill_gemm(sslm_model model, int32_t M, int32_t iters, double* us, int64_t* ops,
                                    int64_t* launches);
/* Per GEMM launch shape: key = class << 56 | M << 40 | N << 20 | K; returns the number of
 * shapes recorded (entries beyond `cap` are not written). */
int sslm_hip_profile_shapes(int64_t* keys, double* ms, int64_t* launches, int64_t* bytes, int64_t* ops, int cap);

/* Per-site trace for bisecting a parity failure (no counterpart in the reference's C ABI; the
 * reference declares the same per-site record, codes and carried scale, in
 * include/superslm/trace_hook.h:36-112 but never installs it from sslm_abi.cpp): after a
 * sslm_decode_step whose sequences ran as one decode unit, the codes and carried scale of row
 * `row` (the row-th sequence of the call) at `site` for the last layer the unit ran --
 * 0 attention RMSNorm, 1 attention context funnel, 2 attention residual, 3 MLP RMSNorm,
 * 4 MLP activation.  With layer_budget 1 every call exposes one layer.  `codes` holds the row
 * (hidden or intermediate size), `scale_me` its (m, e).  Returns the row's length, or -1. */
int32_t sslm_hip_debug_site(sslm_model model, int32_t site, int32_t row, int8_t* codes, int64_t* scale_me);

/* Debug capture of every site of every layer (the records of include/superslm/trace_hook.h:36-112
 * for prefill spans and decode batches alike, which the reference's C ABI never installs).  With
 * max_tokens > 0, every later launch sequence of at most max_tokens tokens (a prefill span, or a
 * decode unit) also writes, per layer it runs, each site's codes and carried scale into a
 * device-side capture area; captured graphs are not used meanwhile.  max_tokens = 0 frees the area
 * and ends the capture.  Sites, in the order of sslm_hip_debug_site's numbering extended:
 * 0 attention RMSNorm, 1 attention context funnel, 2 attention residual, 3 MLP RMSNorm, 4 MLP
 * activation, 5 MLP residual (the committed row), 6 q after RoPE, 7 o_proj funnel, 8 gate funnel,
 * 9 up funnel, 10 down funnel.  sslm_hip_debug_capture_read returns the row of `token` (launch
 * order) at (layer, site) of the last launch sequence that ran that layer: its length (hidden or
 * intermediate size), or -1. */
sslm_status sslm_hip_debug_capture(sslm_model model, int32_t max_tokens);
int32_t sslm_hip_debug_capture_read(sslm_model model, int32_t layer, int32_t site, int32_t token, int8_t* codes,
                                    int64_t* scale_me);

/* The single GEMM + requant of BASELINE configuration 0, on device buffers: int8 A [m, k] x int8
 * W [n, k]^T, int32 accumulate, per-output-row WSC1 fold `fold` [n, 3] (identity, mult, shift),
 * then the per-token dynamic requant funnel with incoming scale `in_m/in_e` and site constant
 * `site_m/site_e` (reference src/matmul.cpp:466-509 + forward_sites.cpp:461-470 +
 * checked_chain_funnel.cpp:257-364).  Writes int8 codes [m, n] and per-row scales
 * out_me[2*t] = m, out_me[2*t+1] = e, and per-row status (0 = Ok, else the reference's
 * SslmForwardStatus value).  All pointers are device pointers; synchronous.  Requires
 * 1 <= m <= 512, k and n multiples of 16, n <= 8192 (else SSLM_INVALID_ARGUMENT). */
sslm_status sslm_hip_gemm_requant(const int8_t* a, const int8_t* w, const int32_t* fold, int32_t m, int32_t n,
                                  int32_t k, int64_t in_m, int64_t in_e, int64_t site_m, int64_t site_e,
                                  int8_t* out_codes, int64_t* out_me, int32_t* out_status);

/* Device memory for callers that hold no HIP runtime of their own (tests, benchmarks): this
 * library's HIP runtime owns the device, so buffers handed to the entry points below come from
 * here.  copy: kind 0 host->device, 1 device->host, 2 device->device; synchronous. */
void* sslm_hip_device_alloc(size_t bytes);
void sslm_hip_device_free(void* p);
sslm_status sslm_hip_copy(void* dst, const void* src, size_t bytes, int kind);
/* Wall-clock-free device synchronisation of the library's streams. */
sslm_status sslm_hip_synchronize(void);

/* Raw int32 GEMM (no epilogue) for verification: out[m, n] = A . W^T, device pointers. */
sslm_status sslm_hip_gemm_i32(const int8_t* a, const int8_t* w, int32_t m, int32_t n, int32_t k, int32_t* out);

/* sslm_hip_gemm_requant for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  No counterpart in the
 * reference.  Same arguments, kernels and results as sslm_hip_gemm_requant, plus `stream` (a
 * hipStream_t; null = the default stream).  It allocates nothing: its scratch (int32 fold
 * outputs, per-tile partial maxima, per-token routing and scales) is one file-scope device array
 * of sslm_hip_noalloc_scratch_bytes() bytes (about 21 MB) that each GPU holds until the process
 * ends.  Asynchronous on `stream`: the outputs are ready once the stream has drained.  Calls on
 * one GPU share that array, so calls that overlap on one GPU (other streams, other threads) race;
 * each call writes every scratch element it reads.  Requires 1 <= m <= SSLM_HIP_NOALLOC_MAX_M,
 * 16 <= n <= SSLM_HIP_NOALLOC_MAX_N, n and k multiples of 16 (else SSLM_INVALID_ARGUMENT, with a
 * message on stderr, and nothing launched).  A launch that fails after the first one was enqueued
 * returns SSLM_HIP_LAUNCH_FAILED (the outputs are then undefined). */
#define SSLM_HIP_LAUNCH_FAILED ((sslm_status)SSLM_STATUS_NEXT_FREE)
#define SSLM_HIP_NOALLOC_MAX_M 128
#define SSLM_HIP_NOALLOC_MAX_N 8192
size_t sslm_hip_noalloc_scratch_bytes(void);
sslm_status sslm_hip_gemm_requant_noalloc(const int8_t* a, const int8_t* w, const int32_t* fold, int32_t m, int32_t n,
                                          int32_t k, int64_t in_m, int64_t in_e, int64_t site_m, int64_t site_e,
                                          int8_t* out_codes, int64_t* out_me, int32_t* out_status, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SSLM_HIP_H */
