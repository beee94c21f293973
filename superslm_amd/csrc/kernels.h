// Kernel-side argument structures and launch wrappers for the SuperSLM HIP backend (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "int_math.h"

namespace sslm {

// Per-token routing for one batched launch.  Decode batches gather one token per sequence;
// a prefill chunk is T tokens of one sequence at consecutive positions.
struct TokenInfo {
	int64_t pos;     // KV position this token lands at (context_length at its start)
	int32_t slot;    // sequence slot: stream state, saturation counter, status
	int32_t block;   // KV pool block of the sequence
};

// Output segment of a fused projection GEMM (q|k|v or gate|up share one launch).
enum SegMode : int32_t { kSegFunnel = 0, kSegWide = 1 };

struct Segment {
	int32_t n_begin, n_end;     // column range in the fused weight matrix
	int32_t mode;               // SegMode
	int32_t ld_out;             // row stride of `out` in elements
	void* out;                  // int32 (funnel, saturated) or int64 (wide) [M, ld_out]
	uint32_t* maxpart;          // funnel: saturating max |value| per (16-column tile, token):
	                            // maxpart[(col / 16) * kPartLd + t]; the consumer reduces the tiles
	const int32_t* fold;        // [n, 3] (identity, mult, shift)
	const int64_t* bias;        // [n] BIA1 codes, or null
	const int8_t* lora_b;       // [n, rank] or null
	const int32_t* lora_dfold;  // [n, 3] (identity, mult, exponent)
	const int8_t* lora_u;       // [M, kMaxRank] adapter intermediate codes of this projection
};

constexpr int kMaxRank = 64;
constexpr int kPartLd = 8192;  // token stride of the per-tile partial maxima (>= tokens per launch)
constexpr int kMaxSeg = 3;
constexpr int kFunnelMaxN = 8192;  // widest row the standalone funnel kernel covers

struct Epilogue {
	Segment seg[kMaxSeg];
	int32_t nseg;
	int32_t rank;
	const int64_t* in_recip;   // [M] reciprocal of the input scale mantissa (bias reconcile)
	const Scale* in_scale;     // [M] input carried scale (bias reconcile exponent)
	const TokenInfo* tok;      // [M]
	int32_t* status;           // [slots] first rejection, (layer << 8) | status
	int32_t layer;
	// logits mode: per (16-column tile, token) argmax keys instead of segments
	unsigned long long* argmax_key;  // [M][key_ld] per (token, 16-column tile) keys, or null
	int32_t key_ld;
	// logits mode: per token a schema mask page (bit j set: token j legal) or null; masked
	// logits count as INT32_MIN (forward_sites.cpp:2443-2449).  Null: no token masked.
	const uint8_t* const* mask_page;
	// raw mode: the int32 accumulator itself, [M, N]
	int32_t* raw_out;
};

// Debug tap (sslm_hip_debug_capture): when `codes` is non-null, a kernel also stores the codes
// [M, n] and carried scales [M] it computed at a site that otherwise stays in registers.
struct SiteTap {
	int8_t* codes;
	Scale* scale;
	int32_t ld;  // row stride of codes
};

struct GemmArgs {
	const int8_t* a;   // [M, K] activation codes, row stride lda
	const int8_t* w;   // [N, K] weights
	// the same weights in the packed decode layout (k_gemv_pk in kernels.hip), or null; decode
	// GEMVs at M <= 32 read them instead of w
	const int8_t* wp;
	int32_t M, N, K, lda;
	Epilogue epi;
	// Decode GEMV split-K: with splits > 1 every split stores its raw int32 partial sums to plane
	// `split` of split_part ([splits][M][N]) and the epilogue is left to the consumer (RawIn).
	int32_t splits;
	int32_t* split_part;
};

// decode GEMV launch shape
struct GemvPlan {
	int tpw;     // 16-column tiles per block
	int splits;  // K splits over gridDim.y
	int cps;     // 128-byte K chunks per split
	int cpw;     // chunks per wave per load batch
	bool wave_tile;  // the wave-per-tile kernel (raw / split planes / argmax at M <= 16)
};
constexpr int kGemvTargetBlocks = 512;

// prefill GEMM launch shape (M > 64)
struct PrefillPlan {
	int bm;      // block rows (256 or 128); block columns are 128
	int splits;  // K splits over gridDim.z (raw partial planes)
	int kspan;   // K per split (multiple of 128)
	int blocks;  // gridDim.x: one tile per block
	bool narrow;  // raw output of the 64 x 64-tile kernel, one plane over the whole K
};
constexpr int kPrefillTargetBlocks = 256;
constexpr int kMaxRawSplits = 8;  // split planes a raw consumer adds

// A projection's output as split-K partial sums whose epilogue (fold, LoRA, bias) the consuming
// row kernel applies: element j of token t is epi_value(epi, t, j, sum_s part[(s * M + t) * ld + j]).
struct RawIn {
	const int32_t* part;  // null: the producer already applied the epilogue
	int32_t splits, ld;
	Epilogue epi;
};

// Status word: the first rejection per sequence slot wins.
__device__ __forceinline__ void set_status(int32_t* status, int32_t slot, int32_t layer, int32_t st) {
	if (st != kOk) atomicCAS(&status[slot], 0, (layer << 8) | st);
}

// Attention runs its heads in parallel, but the reference runs them in order and reports the
// first refusing head: each refusal is recorded as (head << 8) | status with atomicMin, and the
// context funnel that follows resolves the word into the status and resets it.
constexpr int32_t kHeadStatusNone = 0x7fffffff;
__device__ __forceinline__ void report_head(int32_t* head_status, int32_t slot, int32_t head, int32_t st) {
	if (st != kOk) atomicMin(&head_status[slot], (head << 8) | st);
}

}  // namespace sslm

// Host launch wrappers (kernels.hip).
namespace sslm_launch {
using namespace sslm;

// Thrown by a launch wrapper, before anything is enqueued, when a launch does not fit any kernel
// it has (a GEMM without a complete output, a row no instance covers).  Such a launch is a bug of
// the caller; the runtime's entry points catch it and return a status instead of launching.
struct LaunchRefused {
	const char* what;
};

void gemm(const GemmArgs& g, hipStream_t s);
// launch shape of the decode GEMV (M <= 64, K % 128 == 0); `split_ok`: the caller consumes raw
// split-K partials; `raw_or_argmax`: no projection epilogue in the kernel (raw accumulators or
// argmax keys)
GemvPlan gemv_plan(int M, int N, int K, bool split_ok, bool raw_or_argmax = false);
bool gemv_eligible(int M, int K);
// Split-K planes a raw decode GEMV writes for a consumer that adds them: the packed kernels' plan
// when g.wp is set and they take the launch, else gemv_plan's.  1 = a single plane.
int gemv_raw_splits(const GemmArgs& g);
// bytes of the packed decode copy of an [N, K] matrix (whole 16-row tiles)
size_t packed_bytes(int N, int K);
// writes the packed decode copy of w [N, K] (K % 128 == 0) into wp
void pack_gemv(const int8_t* w, int N, int K, int8_t* wp, hipStream_t s);
bool wide_gemm_ok(const GemmArgs& g);  // the prefill launch takes the 256 x 160-tile kernel
// launch shape of the prefill GEMM; `split_ok` as for gemv_plan
PrefillPlan prefill_plan(int M, int N, int K, bool split_ok);
// the MFMA prefill GEMM takes K in multiples of its 128-deep step; other K use the tiled kernel
bool prefill_mfma_k(int K);

struct RowNormArgs {
	// input stream codes: in_codes[idx[t] * ld_in], input scale ignored (norm kills it)
	const int8_t* in_codes;
	const int32_t* in_idx;
	int32_t ld_in;
	const int32_t* gain;  // [H]
	Scale site;
	int8_t* out;          // [M, H]
	Scale* out_scale;     // [M]
	int64_t* out_recip;   // [M] reciprocal(out_scale.m), for bias reconcile downstream
};

void embed(const int32_t* tokens, int M, const int8_t* embed_w, int H, int vocab, Scale site, int8_t* out_codes,
           const int32_t* out_idx, Scale* out_scale, const int32_t* scale_idx, const TokenInfo* tok,
           int32_t* status, hipStream_t s);

// attention-input side: q funnel + RoPE(q); K/V landing + RoPE(K) into the KV pool
struct QkvPostArgs {
	int M, H, NH, NKV, D;
	int64_t cap;
	const TokenInfo* tok;
	const int32_t* q_f;       // [M, H] funnel-mode q fold outputs
	const uint32_t* q_maxpart;  // tiles [0, H/16) of the q|k|v projection
	RawIn raw;                  // or: raw q|k|v partials (q_f, q_maxpart and kv_f unused)
	const int64_t* kv_f;      // [M, 2*NKV*D] k then v wide values
	const Scale* in_scale;    // [M] normed scale (landing operand and q's incoming)
	Scale q_site;
	const int64_t* r_t_k;     // [NKV]
	const int64_t* e_t_k;
	const int64_t* r_t_v;
	const int64_t* e_t_v;
	const int64_t* rope_cos;  // [cap, D/2]
	const int64_t* rope_sin;
	int8_t* kv_pool;
	int64_t block_bytes;
	int32_t layer;
	int8_t* q_rot;            // [M, H]
	Scale* q_scale;           // [M]
	unsigned long long* sat;  // [slots]
	int32_t* status;
	// Staged landing (prefill spans): when set, the landed K/V codes go to kv_stage
	// ([M][K heads | V heads][D]) and the clamp counts to sat_stage[M] instead of the pool and
	// `sat`; kv_commit() then writes them once every token's q funnel has passed.
	int8_t* kv_stage;
	uint32_t* sat_stage;
};
void qkv_post(const QkvPostArgs& a, hipStream_t s);
// Writes the staged K/V rows of a prefill span into the pool and adds the clamp counts, unless
// the slot's status holds a refusal; always clears sat_stage.
void kv_commit(const QkvPostArgs& a, hipStream_t s);

struct AttnArgs {
	int M, H, NH, NKV, D;
	int64_t cap;
	const TokenInfo* tok;
	const int8_t* q_rot;      // [M, H] (attention: rotated q codes from qkv_post)
	const Scale* q_scale;     // [M]
	const int64_t* khead_m;   // [NKV]
	const int64_t* khead_e;
	const int32_t* ctx_fold;  // [NH, 3]
	int8_t* kv_pool;
	int64_t block_bytes;
	int32_t layer;
	int64_t ln2_q, b_q, ca_q;
	int32_t* ctx_f;           // [M, H]
	uint32_t* ctx_maxpart;    // [NH * kPartLd]: one partial per query head
	int64_t* scratch;         // [M, NH, cap] when rows exceed LDS
	int32_t* status;
	int32_t* head_status;     // [slots] attention-stage refusals, (head << 8) | status, min wins
	// attention_decode only: the q|k|v post-processing inputs (funnel-epilogue outputs of the
	// projection), in place of q_rot / q_scale
	const int32_t* q_f;         // [M, H]
	const uint32_t* q_maxpart;  // tiles [0, H/16)
	const int64_t* kv_f;        // [M, 2*NKV*D] k then v
	const Scale* in_scale;      // [M] normed scale
	Scale q_site;
	const int64_t* r_t_k;       // [NKV]
	const int64_t* e_t_k;
	const int64_t* r_t_v;
	const int64_t* e_t_v;
	const int64_t* rope_cos;    // [cap, D/2]
	const int64_t* rope_sin;
	unsigned long long* sat;    // [slots]
	SiteTap q_tap;              // attention_decode: the rotated q codes of each head, and the q scale
	int32_t wcap;               // attention_decode: score rows of the grouped kernel, a multiple of 128
	                            // at least every width (pos + 1) of the launch (group_width_cap)
	int32_t row_halves;         // attention_decode, grouped kernel: 1, or 2 blocks per (token, KV group)
};
// The grouped decode kernel's score-row length for a launch whose widest row is `max_width`:
// rounded up to 512 (so a decode graph keyed by it is re-recorded once per 512 positions), at
// most the cap rounded up to 128.
inline int32_t group_width_cap(int64_t max_width, int64_t cap) {
	const int64_t b = (max_width + 511) / 512 * 512, c = (cap + 127) / 128 * 128;
	return (int32_t)(b < c ? b : c);
}
// `one_sequence`: the launch holds one sequence's consecutive positions (a prefill chunk), so
// the query-tiled kernel may run (unless SSLM_HIP_TILED_ATTN=0).
void attention(const AttnArgs& a, hipStream_t s, bool one_sequence = false);
bool tiled_attention_enabled();
// Decode attention with the q|k|v post-processing fused in (one block per (query head, token)):
// valid when every token of the launch belongs to a different sequence, so no token attends to
// a position another block of the launch writes.
void attention_decode(const AttnArgs& a, hipStream_t s);
// attention_decode runs one block per (token, KV head) for this launch shape when the shape fits
// (SSLM_HIP_GROUPED_ATTN=1 forces it wherever it fits, =0 turns it off)
bool grouped_attention_chosen(int M, int NKV, int64_t cap);
// blocks per (token, KV group) of the grouped decode attention: 2 splits the group's query heads
// in halves (SSLM_HIP_GROUP_HALVES=1|2 overrides)
int group_row_halves(int M, int NKV, int G);
// Queries and sets the grouped decode kernel's LDS attributes for head size D and group size G
// (once per process; call before any capture).  False when the runtime refuses them.
bool attention_prepare(int D, int G);
// the attention row (cap int64 values) lives in LDS up to this context capacity, else in
// AttnArgs::scratch ([M, NH, cap] int64)
constexpr int64_t kAttnLdsCap = 6144;
inline bool attention_in_lds(int64_t cap) { return cap <= kAttnLdsCap; }

// funnel over an int32 fold-output row; `incoming` per token or null (empty span, the attn_ctx site)
struct FunnelArgs {
	int M, N;
	const TokenInfo* tok;
	const int32_t* f;
	int32_t ld_f;
	const uint32_t* maxpart;  // [ntiles * kPartLd]
	int32_t ntiles;
	const Scale* incoming;
	Scale site;
	int8_t* out;
	Scale* out_scale;
	int32_t layer;
	int32_t* status;
	int32_t* head_status;  // or null: attention-stage refusals to resolve into `status` first
};
void funnel(const FunnelArgs& a, hipStream_t s);

// o funnel -> attn residual -> mlp RMSNorm   /  down funnel -> mlp residual (commit) -> next norm
struct ResidualArgs {
	int M, H;
	const TokenInfo* tok;
	const int32_t* branch_f;   // [M, H] funnel-mode fold outputs of o_proj / down_proj
	const uint32_t* branch_maxpart;  // tiles [0, H/16)
	RawIn raw;                       // or: raw projection partials (branch_f, branch_maxpart unused)
	const Scale* branch_in;    // [M] incoming scale of the projection (ctx / act)
	Scale branch_site;
	int8_t* stream;            // stream codes, row stream_idx[t]
	const int32_t* stream_idx;
	Scale* stream_scale;       // row stream_idx[t]
	Scale res_site;
	int8_t* out_stream;        // residual output codes, row out_idx[t]
	const int32_t* out_idx;
	Scale* out_stream_scale;   // row out_idx[t]
	const int32_t* gain;       // next RMSNorm (null = none)
	Scale norm_site;
	int8_t* norm_out;          // [M, H]
	Scale* norm_scale;         // [M]
	int64_t* norm_recip;       // [M]
	int32_t layer;
	int32_t* status;
	SiteTap branch_tap;        // the projection funnel's codes (o / down) and scale
};
void residual_norm(const ResidualArgs& a, hipStream_t s);

void rmsnorm(const RowNormArgs& a, int M, int H, const TokenInfo* tok, int32_t* status, int32_t layer,
             hipStream_t s);

// gate/up funnels -> SiLU LUT product -> act funnel
struct ActArgs {
	int M, I;
	const TokenInfo* tok;
	const int32_t* gu_f;     // [M, 2I] gate then up
	const uint32_t* gu_maxpart;  // tiles [0, I/16) gate, [I/16, 2I/16) up
	RawIn raw;                   // or: raw gate|up partials (gu_f, gu_maxpart unused)
	const Scale* in_scale;   // [M] mlp-normed scale (incoming of gate and up)
	Scale gate_site, up_site, act_site;
	const int32_t* silu;     // [1025]
	int8_t* act;             // [M, I]
	Scale* act_scale;        // [M]
	int32_t layer;
	int32_t* status;
	// sliced form (decode rows, funnel-epilogue input): the SiLU products, per-slice maxima and
	// the gate / up scales between its two kernels
	int32_t* prod;           // [M, I]
	uint32_t* act_maxpart;   // [kMaxActSlices * kPartLd]
	Scale* gu_scale;         // [M, 2] gate, up
	SiteTap gate_tap, up_tap;  // the gate / up funnels' codes and scales
};
constexpr int kMaxActSlices = 16;
constexpr int kMaxSlicedActRows = 64;  // rows the sliced form's buffers hold
void mlp_act(const ActArgs& a, hipStream_t s);
// The same step on every row cut into column slices, one block per (row, slice), in two
// launches: gate and up funnels, SiLU products and per-slice maxima; then the act funnel over the
// slices' maxima and the codes.  For short batches (decode), whose one block per row would leave
// most CUs idle; requires the funnel-epilogue input (tile maxima, no raw planes) and
// M <= kMaxSlicedActRows.
bool mlp_act_sliced_ok(const ActArgs& a);
void mlp_act_sliced(const ActArgs& a, hipStream_t s);

// whether the row kernels' register tiling covers this geometry
bool row_geometry_ok(int H, int I, int NKV, int D);

// LoRA intermediate u = clamp(amp_fold(A x)) for up to 3 projections sharing one input
struct LoraUArgs {
	int M, K, rank, nproj;
	const int8_t* x;  // [M, K]
	const int8_t* a[3];       // [rank, K]
	const int32_t* ufold[3];  // [rank, 3]
	int8_t* u[3];             // [M, kMaxRank]
};
void lora_u(const LoraUArgs& a, hipStream_t s);

// Snapshot (or restore) of what one decode launch sequence changes for each of its tokens: the
// slot's stream row (H codes), scale and clamp counter, and the K/V rows of layers [l0, l1) at
// the token's position.
struct SlotCopyArgs {
	const TokenInfo* tok;  // [n]
	int8_t* codes;         // [slots, H]
	Scale* scale;
	unsigned long long* sat;
	int8_t* snap_codes;    // [slots, H]
	Scale* snap_scale;
	unsigned long long* snap_sat;
	int8_t* kv_pool;
	int64_t block_bytes, cap;
	int32_t H, NKV, D, l0, l1;
	int8_t* snap_kv;       // [slots, snap_kv_ld]: layer l's K then V rows at l * 2 * NKV * D
	int64_t snap_kv_ld;
};
void slot_state_copy(const SlotCopyArgs& a, int n, bool restore, hipStream_t s);

// per-tile argmax keys -> token ids (lowest index among equal maxima)
// Bench reference: one streaming read of `bytes` bytes (a multiple of 16) of device memory.
void stream_read(const void* p, int64_t bytes, int* sink, hipStream_t s);
// Debug capture: rows t < M of src (row idx[t], or t when idx is null) of n codes and their scales
// into dst[t * ld] / sdst[t].
void debug_gather(const int8_t* src, const Scale* ssrc, const int32_t* idx, int n, int M, int8_t* dst, Scale* sdst,
                  int ld, hipStream_t s);
void argmax_finalize(const unsigned long long* keys, int ntiles, int M, int32_t* out_tokens, hipStream_t s);

// Damped greedy's candidate set on the device: per row of raw logits [M][V] (masked logits, per
// the row's mask page, count as INT32_MIN), the k entries first in the order (logit descending,
// legal before masked, index ascending), written unordered as (index, logit) pairs to
// out[row * k ..].  k <= kTopKMax.
constexpr int kTopKMax = 1024;
void topk_candidates(const int32_t* logits, int V, int M, const uint8_t* const* mask_page, int k, int2* out,
                     hipStream_t s);

}  // namespace sslm_launch
