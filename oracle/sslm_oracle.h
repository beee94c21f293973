/* CPU restatement of SuperSLM's integer forward path -- TEST INFRASTRUCTURE ONLY.
 *
 * This library is the parity oracle for the HIP backend under superslm_amd/.  Only the
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and only as the
 * checker.  The product path never links or calls it.
 *
 * Every function restates the reference algorithm (file:line cited at each definition in
 * sslm_oracle.c) in plain C11 with gcc's __int128 for the wide intermediates.  Pinning:
 *   - primitives: against the reference's golden fixture vectors (JSON files under tests/golden,
 *     extracted from the reference tests/ fixture headers) and against closed forms
 *     (exact 128-bit division for the reciprocal, r*r <= n < (r+1)^2 for isqrt, brute force);
 *   - sites and layer loops: against the compiled reference (oracle/_ref) on seeded
 *     synthetic artifacts, token for token and KV byte for KV byte.
 */
#ifndef SSLM_ORACLE_H
#define SSLM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* reference include/superslm/checked_chain_funnel.h:56 CarriedScale */
typedef struct or_scale {
	int64_t m;
	int64_t e;
} or_scale;

/* reference include/superslm/checked_chain_funnel.h:68-284 SslmForwardStatus (same order) */
enum or_status {
	OR_OK = 0,
	OR_CHAIN_INPUT_OUT_OF_DOMAIN,
	OR_LOGIT_NARROWING_OVERFLOW,
	OR_IEXP_CONSTANTS_OUT_OF_DOMAIN,
	OR_CARRIED_SCALE_MANTISSA_OUT_OF_DOMAIN,
	OR_SILU_COMPOSITION_SCALE_OUT_OF_DOMAIN,
	OR_RDBPOT_EXPONENT_OUT_OF_DOMAIN,
	OR_SOFTMAX_ROW_WIDTH_OUT_OF_DOMAIN,
	OR_TOKEN_ID_OUT_OF_RANGE,
	OR_POSITION_OVER_CAP,
	OR_WORKSPACE_TOO_SMALL,
	OR_KV_CAPACITY_EXHAUSTED,
	OR_KV_PRECISION_UNSUPPORTED,
	OR_INVALID_LAYER_BUDGET,
	OR_ROPE_TABLE_TENSOR_MISSING,
	OR_ROPE_TABLE_EXTENT_EXCEEDED,
	OR_INVALID_CONTEXT_CAP,
	OR_HEAD_DIM_GEOMETRY_MISMATCH,
	OR_KV_HEAD_GEOMETRY_MISMATCH,
	OR_SEQUENCE_ALREADY_COMPLETE,
	OR_SOFTMAX_KERNEL_REFUSED_AFTER_GATE_ACCEPTED,
	OR_RESIDUAL_RECONCILIATION_MAGNITUDE_OUT_OF_DOMAIN,
	OR_INVALID_HIDDEN_CODES,
	OR_IEXP_SCALE_DERIVATION_OUT_OF_DOMAIN,
	OR_BIAS_RECONCILE_PRODUCT_OUT_OF_DOMAIN,
};

/* One LoRA projection (reference include/superslm/forward_sites.h:593-607).  a: int8 [rank, in],
 * b: int8 [out, rank], u_fold: int32 [rank, 3], d_fold: int32 [out, 3] (identity, mult, exponent). */
typedef struct or_lora_proj {
	const int8_t* a;
	const int8_t* b;
	const int32_t* u_fold;
	const int32_t* d_fold;
} or_lora_proj;

/* Projection order used by every per-projection array below. */
enum { OR_Q = 0, OR_K, OR_V, OR_O, OR_GATE, OR_UP, OR_DOWN, OR_NPROJ };

/* One layer's weights and constants (reference include/superslm/forward_sites.h:609-747
 * LayerWeights, marshalled as include/superslm/layer_marshal.h:141-330 does). */
typedef struct or_layer {
	const int8_t* w[OR_NPROJ];      /* int8 [N, K] row-major (nn.Linear) */
	const int32_t* fold[OR_NPROJ];  /* int32 [N, 3] WSC1 (identity, mult, shift) */
	const int32_t* ctx_fold;        /* int32 [num_heads, 3] */
	const int64_t* bias[3];         /* q, k, v BIA1 int64 [N]; NULL when absent */
	const int32_t* attn_gain;       /* int32 [H], the int8 gain sign-extended */
	const int32_t* mlp_gain;
	const int64_t* kv_r_t_k;        /* [NKV] KvLandingReciprocals word 2 */
	const int64_t* kv_e_t_k;        /* [NKV] word 1 */
	const int64_t* kv_r_t_v;
	const int64_t* kv_e_t_v;
	const int64_t* khead_m;         /* [NKV] softmax_khead (m, e) */
	const int64_t* khead_e;
	or_scale attn_norm_sc, q_sc, ctx_sc, o_sc, attn_res_sc;
	or_scale mlp_norm_sc, gate_sc, up_sc, act_sc, down_sc, mlp_res_sc;
	uint32_t lora_rank;                 /* 0 = no adapter */
	const or_lora_proj* lora[OR_NPROJ]; /* NULL entries = projection unadapted */
} or_layer;

typedef struct or_model {
	uint32_t hidden, layers, heads, kv_heads, head_dim, inter, vocab;
	int64_t context_cap;
	const or_layer* layer;
	const int8_t* embed;        /* [V, H] */
	const int8_t* head;         /* [V, H] (the embed table when tied) */
	const int32_t* final_gain;  /* [H] */
	or_scale embed_sc, final_sc;
	const int64_t* rope_cos;    /* [cap, D/2] Q2.30 */
	const int64_t* rope_sin;
	const int32_t* silu_table;  /* [1025] */
} or_model;

/* reference include/superslm/forward_sites.h:431-454 SequenceLayerState */
typedef struct or_seq {
	int8_t* hidden;
	or_scale scale;
	uint32_t layer_index;
	uint64_t kv_saturation_count;
	int64_t context_length;
} or_seq;

/* ---- primitives (src/intmath.cpp) ---- */
int32_t or_srdhm(int32_t a, int32_t b);
int32_t or_rdbpot32(int32_t x, int exponent);
int64_t or_rdbpot64(int64_t x, int exponent);
int32_t or_mbqm(int32_t x, int32_t mult, int shift);
int32_t or_sat_shl32(int32_t x, int shift);
int or_clz64(uint64_t n);
int64_t or_max_abs_wide(const int64_t* x, size_t n);
int64_t or_normalize_scale(int64_t d_prime, int* out_s);
int64_t or_reciprocal(int64_t dn);
int8_t or_requant_code_wide(int64_t x, int64_t r, int s);
int64_t or_isqrt(int64_t n);
int or_iexp_construct(int64_t q, int64_t q_ln2, int64_t q_b, int64_t q_c, int64_t* z, int64_t* base);
int64_t or_iexp_evaluate(int64_t z, int64_t base, int64_t q_c);
int or_iexp_scale_constants(int64_t m, int64_t e, int64_t ln2_q, int ln2_fmt, int64_t b_q, int b_fmt,
                            int64_t ca_q, int ca_fmt, int64_t* q_ln2, int64_t* q_b, int64_t* q_c);
void or_rope_pair(int32_t x, int32_t y, int32_t c, int32_t s, int64_t* out_x, int64_t* out_y);
int or_softmax_row_q15(const int64_t* scores, size_t width, int64_t q_ln2, int64_t q_b, int64_t q_c,
                       int64_t* out_probs);
int or_bias_reconcile_wide(int64_t b, int64_t q_b, int64_t r_a, int64_t e_a, int64_t* out);
int32_t or_silu_sigmoid_q15(const int32_t* table, int8_t code, int64_t m, int e);
void or_iexp_pinned(int64_t* ln2_q, int64_t* b_q, int64_t* ca_q);

/* ---- funnel + sites (src/forward) ---- */
or_scale or_combine_scale(or_scale a, or_scale b);
int or_requant_chain(const int64_t* row, size_t n, const or_scale* incoming, size_t n_in, or_scale site,
                     int8_t* out_codes, or_scale* out_scale);
int or_check_softmax_width(int64_t q_b, int64_t q_c, size_t width);
int64_t or_apply_fold(int64_t acc, int32_t identity, int32_t mult, int32_t shift);
int64_t or_apply_amp_fold(int64_t acc, int32_t identity, int32_t mult, int32_t exponent);
int64_t or_landing_rescale(int64_t branch, int64_t m_a, int64_t r_t, int64_t e_a, int64_t e_t,
                           uint64_t* sat_count, int* exceeded_i64);
int or_rmsnorm_site(const int8_t* h, const int32_t* g, size_t n, or_scale site, int8_t* out,
                    or_scale* out_scale);
int or_embed_entry(const or_model* m, int32_t token, int8_t* out, or_scale* out_scale);
int or_mlp_act_site(const int8_t* gate, or_scale gs, const int8_t* up, or_scale us, size_t n,
                    const int32_t* table, or_scale site, int8_t* out, or_scale* out_scale);
int or_residual_site(const int8_t* branch, or_scale bs, const int8_t* stream, or_scale ss, size_t n,
                     or_scale site, int8_t* out, or_scale* out_scale);
/* GEMM -> fold -> LoRA -> bias -> funnel for one row (forward_sites.cpp:1114-1154). */
int or_project_row(const int8_t* x, or_scale in_scale, size_t in_ch, size_t out_ch, const int8_t* w,
                   const int32_t* fold, const int64_t* bias, const or_lora_proj* lora, uint32_t rank,
                   or_scale site, int8_t* out, or_scale* out_scale);
void or_gemm_i8(const int8_t* a, const int8_t* w, size_t m, size_t k, size_t n, int64_t* out);

/* ---- layer loops + head ---- */
size_t or_kv_block_bytes(const or_model* m);
int or_run_layer_loop(const or_model* m, or_seq* seq, uint32_t layer_budget, int8_t* kv);
int or_run_chunk(const or_model* m, int8_t* hidden_chunk, or_scale* scales, size_t tokens,
                 int64_t ctx_start, int8_t* kv, uint64_t* sat_count);
int or_final_logits(const or_model* m, const int8_t* hidden, int32_t* out_logits);
int32_t or_argmax(const int32_t* logits, size_t n);

/* Per-site trace of the layer loops (the instrument the reference declares in
 * include/superslm/trace_hook.h:36-112 -- per site and token the codes and the carried scale):
 * when set, or_run_layer_loop calls `fn` after each listed site of every layer it runs, and
 * or_run_chunk after each site of every layer, once per token in position order (its sites run
 * over the whole chunk, as forward_sites.cpp:2098-2410 does).  One process-wide hook: test
 * infrastructure, single-threaded use only. */
enum {
	OR_SITE_ATTN_NORM = 0,
	OR_SITE_CTX = 1,
	OR_SITE_ATTN_RESIDUAL = 2,
	OR_SITE_MLP_NORM = 3,
	OR_SITE_ACT = 4,
	OR_SITE_MLP_RESIDUAL = 5,
	OR_SITE_Q = 6,
	OR_SITE_O = 7,
	OR_SITE_GATE = 8,
	OR_SITE_UP = 9,
	OR_SITE_DOWN = 10,
	OR_SITE_Q_ROT = 11 /* q after RoPE (no reference site; checks the backends' fused q landing) */
};
typedef void (*or_trace_fn)(void* user, uint32_t layer, int site, const int8_t* codes, size_t n, int64_t scale_m,
                            int64_t scale_e);
void or_set_trace(or_trace_fn fn, void* user);

#ifdef __cplusplus
}
#endif

#endif
