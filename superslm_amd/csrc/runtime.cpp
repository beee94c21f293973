// Host runtime of the HIP backend: model residency, KV pool, sequences, and the orchestration
// of the integer forward (layer-sliced decode and chunked prefill) behind the sslm_* C ABI.
//
// Semantics follow the reference CPU path:
//   sslm_prefill        src/sslm_abi.cpp:1417-1567, :1950-1972
//   sslm_decode_step    src/sslm_abi.cpp:1989-2434
//   layer loop          src/forward/forward_sites.cpp:1429-2014 (decode), :2098-2401 (prefill)
// A decode call batches every sequence that sits at the same layer into one launch sequence;
// a prefill call runs its admitted tokens as chunks of at most kMaxTokens through every layer.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <memory>
#include <mutex>
#include <set>
#include <string>
#include <vector>

#include "../../include/sslm_hip.h"
#include "artifact.h"
#include "kernels.h"

using namespace sslm;

namespace {

constexpr int kMaxTokens = 512;      // tokens per launch sequence (prefill chunk / decode group)
constexpr int kSlotCapacity = 1024;  // live sequences per model

struct HipError {
	hipError_t e;
};

inline void ck(hipError_t e) {
	if (e != hipSuccess) throw HipError{e};
}

template <typename T>
T* dalloc(size_t n, std::vector<void*>* owned) {
	void* p = nullptr;
	ck(hipMalloc(&p, n * sizeof(T) + 16));
	ck(hipMemset(p, 0, n * sizeof(T) + 16));
	owned->push_back(p);
	return (T*)p;
}

template <typename T>
T* dupload(const std::vector<T>& v, std::vector<void*>* owned) {
	T* p = dalloc<T>(v.size(), owned);
	if (!v.empty()) ck(hipMemcpy(p, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice));
	return p;
}

// ------------------------------------------------------------------------------------------
// profiling: events around launches, accumulated per class
// ------------------------------------------------------------------------------------------
struct ProfState {
	bool on = false;
	double ms[SSLM_HIP_PROFILE_CLASSES] = {0};
	int64_t launches[SSLM_HIP_PROFILE_CLASSES] = {0};
	int64_t bytes[SSLM_HIP_PROFILE_CLASSES] = {0};
	int64_t ops[SSLM_HIP_PROFILE_CLASSES] = {0};
	struct Pending {
		hipEvent_t a, b;
		int cls;
	};
	std::vector<Pending> pending;
	std::vector<hipEvent_t> pool;
	std::mutex mu;
};
ProfState g_prof;

hipEvent_t prof_event() {
	if (!g_prof.pool.empty()) {
		hipEvent_t e = g_prof.pool.back();
		g_prof.pool.pop_back();
		return e;
	}
	hipEvent_t e;
	ck(hipEventCreate(&e));
	return e;
}

struct ProfScope {
	hipStream_t s;
	int cls;
	hipEvent_t a = nullptr;
	ProfScope(hipStream_t s_, int c, int64_t bytes, int64_t ops) : s(s_), cls(c) {
		if (!g_prof.on) return;
		a = prof_event();
		ck(hipEventRecord(a, s));
		g_prof.bytes[c] += bytes;
		g_prof.ops[c] += ops;
		g_prof.launches[c] += 1;
	}
	~ProfScope() {
		if (!a) return;
		hipEvent_t b = prof_event();
		(void)hipEventRecord(b, s);
		g_prof.pending.push_back({a, b, cls});
	}
};

void prof_collect() {
	if (g_prof.pending.empty()) return;
	for (auto& p : g_prof.pending) {
		(void)hipEventSynchronize(p.b);
		float ms = 0;
		(void)hipEventElapsedTime(&ms, p.a, p.b);
		g_prof.ms[p.cls] += ms;
		g_prof.pool.push_back(p.a);
		g_prof.pool.push_back(p.b);
	}
	g_prof.pending.clear();
}

enum ProfClass { kProfGemm = 0, kProfHead = 1, kProfAttn = 2, kProfRow = 3, kProfLora = 4 };

}  // namespace

// ------------------------------------------------------------------------------------------
// handle types
// ------------------------------------------------------------------------------------------
struct DevLayer {
	int8_t *w_qkv, *w_o, *w_gu, *w_down;
	int32_t *f_qkv, *f_o, *f_gu, *f_down, *ctx_fold;
	int64_t *b_q, *b_k, *b_v;
	int32_t *attn_gain, *mlp_gain;
	int64_t *r_t_k, *e_t_k, *r_t_v, *e_t_v, *khead_m, *khead_e;
	Scale attn_norm, q, ctx, o, attn_res, mlp_norm, gate, up, act, down, mlp_res;
};

struct AdapterProj {
	int8_t* a = nullptr;       // [rank, K]
	int8_t* b = nullptr;       // [N, rank]
	int32_t* ufold = nullptr;  // [rank, 3]
	int32_t* dfold = nullptr;  // [N, 3]
};

struct sslm_adapter_s {
	sslm_model model = nullptr;
	uint32_t rank = 0;
	std::vector<AdapterProj> proj;  // [layer * 7 + p], order q k v o gate up down
	std::vector<void*> owned;
	size_t bytes = 0;
	std::atomic<int> live_refs{0};
};

struct sslm_model_s {
	Artifact art;
	ModelConfig c;
	int H, L, NH, NKV, D, I, V, KVH;
	int64_t cap;
	size_t block_bytes;
	hipStream_t stream = nullptr;
	std::vector<void*> owned;
	std::vector<DevLayer> layers;
	int8_t *embed, *head;
	int32_t *final_gain, *silu;
	int64_t *rope_cos, *rope_sin;
	Scale embed_site, final_site;
	int64_t ln2_q, b_q, ca_q;
	// per-slot sequence state
	int8_t* stream_codes;   // [kSlotCapacity, H]
	Scale* stream_scale;    // [kSlotCapacity]
	unsigned long long* sat;  // [kSlotCapacity]
	int32_t* status;        // [kSlotCapacity]
	std::vector<int> free_slots;
	// launch workspace (kMaxTokens rows)
	TokenInfo* tok;
	int32_t *tok_ids, *ident, *slot_idx, *out_tokens;
	int8_t *hid_chunk, *normed, *q_rot, *ctx, *attn_stream, *mlp_normed, *act, *final_codes;
	Scale *hid_chunk_scale, *normed_scale, *q_scale, *ctx_scale, *attn_stream_scale, *mlp_scale, *act_scale,
	    *final_scale;
	int64_t *normed_recip, *mlp_recip, *kv_f, *attn_scratch;
	int32_t *q_f, *ctx_f, *o_f, *gu_f, *down_f;
	uint32_t *mx_q, *mx_ctx, *mx_o, *mx_gu, *mx_down;  // per (16-column tile, token) partial maxima
	unsigned long long* argmax_key;
	int32_t* raw_part;  // decode GEMV split-K partial planes, consumed by the next row kernel
	int8_t* lora_u[3];
	int8_t* pool_dev = nullptr;  // KV pool of the launch sequence being recorded
	std::atomic<int> live_refs{0};
	std::mutex mu;  // serializes GPU submission on this model
};

struct sslm_kv_pool_s {
	sslm_model model = nullptr;
	void* buf = nullptr;
	size_t buf_size = 0;
	uint32_t block_count = 0;
	size_t block_size = 0;
	int8_t* dev = nullptr;
	std::vector<uint32_t> free_list;
	std::atomic<int> live_refs{0};
	std::mutex mu;
};

struct sslm_seq_s {
	sslm_model model = nullptr;
	sslm_kv_pool pool = nullptr;
	uint32_t block = 0;
	int slot = -1;
	uint32_t layer_index = 0;
	int64_t context_length = 0;
	int32_t current_token = -1;
	bool ready_for_logits = false;
	sslm_adapter adapter = nullptr;
	std::mutex mu;
};

struct sslm_workspace_s {
	void* buf = nullptr;
	size_t buf_size = 0;
	sslm_config config{};
};

namespace {

std::mutex g_registry_mu;
std::set<sslm_seq_s*> g_live_seqs;

// ------------------------------------------------------------------------------------------
// launch helpers
// ------------------------------------------------------------------------------------------
GemmArgs gemm_args(sslm_model m, const int8_t* a, int M, int lda, const int8_t* w, int N, int K) {
	GemmArgs g{};
	g.a = a;
	g.w = w;
	g.M = M;
	g.N = N;
	g.K = K;
	g.lda = lda;
	g.epi.tok = m->tok;
	g.epi.status = m->status;
	return g;
}

Segment funnel_seg(int n0, int n1, int32_t* out, int ld, uint32_t* mx, const int32_t* fold, const int64_t* bias) {
	Segment s{};
	s.n_begin = n0;
	s.n_end = n1;
	s.mode = kSegFunnel;
	s.out = out;
	s.ld_out = ld;
	s.maxpart = mx;
	s.fold = fold;
	s.bias = bias;
	return s;
}

void run_gemm(sslm_model m, const GemmArgs& g, int cls) {
	const int64_t out_bytes = g.epi.argmax_key ? 0 : (int64_t)g.M * g.N * 4;
	ProfScope p(m->stream, cls, (int64_t)g.N * g.K + (int64_t)g.M * g.K + 12LL * g.N + out_bytes,
	            2LL * g.M * g.N * g.K);
	sslm_launch::gemm(g, m->stream);
	ck(hipGetLastError());
}

// Decode projections whose GEMV splits K hand their raw partial planes to the next row kernel,
// which applies the epilogue; call once g.epi is complete.  Returns a null RawIn otherwise.
// `allow`: the consumer's raw variant holds its row in registers without spilling.
RawIn split_raw(sslm_model m, GemmArgs& g, bool allow) {
	RawIn r{};
	if (!allow || !m->raw_part) return r;
	bool lora = false;
	for (int i = 0; i < g.epi.nseg; ++i) lora = lora || g.epi.seg[i].lora_b;
	int splits = 1;
	if (sslm_launch::gemv_eligible(g.M, g.K)) splits = sslm_launch::gemv_plan(g.M, g.N, g.K, true).splits;
	else if (!lora && g.K % 64 == 0) splits = sslm_launch::prefill_plan(g.M, g.N, g.K, true).splits;
	if (splits <= 1) return r;
	g.splits = splits;
	g.split_part = m->raw_part;
	r.part = m->raw_part;
	r.splits = splits;
	r.ld = g.N;
	r.epi = g.epi;
	return r;
}

void attach_lora(sslm_model m, sslm_adapter ad, int layer, int proj, Segment* seg, int slot_u) {
	if (!ad) return;
	const AdapterProj& p = ad->proj[(size_t)layer * 7 + proj];
	if (!p.a) return;
	seg->lora_b = p.b;
	seg->lora_dfold = p.dfold;
	seg->lora_u = m->lora_u[slot_u];
}

void run_lora_u(sslm_model m, sslm_adapter ad, int layer, const int* projs, int n, const int8_t* x, int M, int K) {
	if (!ad) return;
	sslm_launch::LoraUArgs a{};
	a.M = M;
	a.K = K;
	a.rank = (int)ad->rank;
	a.x = x;
	int cnt = 0;
	for (int i = 0; i < n; ++i) {
		const AdapterProj& p = ad->proj[(size_t)layer * 7 + projs[i]];
		if (!p.a) continue;
		a.a[cnt] = p.a;
		a.ufold[cnt] = p.ufold;
		a.u[cnt] = m->lora_u[i];
		++cnt;
	}
	if (!cnt) return;
	a.nproj = cnt;
	ProfScope ps(m->stream, kProfLora, (int64_t)cnt * ad->rank * K + (int64_t)M * K, 2LL * M * cnt * ad->rank * K);
	sslm_launch::lora_u(a, m->stream);
	ck(hipGetLastError());
}

// The stream (committed hidden state) a launch sequence reads and commits: decode batches use the
// per-slot state, prefill chunks the chunk rows.
struct StreamRef {
	int8_t* codes;
	Scale* scale;
	const int32_t* idx;
};

// Layers [l0, l1) for M tokens whose TokenInfo is already on the device.
void run_layers(sslm_model m, int M, StreamRef st, int l0, int l1, sslm_adapter ad) {
	const int H = m->H, I = m->I, KVH = m->KVH;
	hipStream_t s = m->stream;
	{
		ProfScope p(s, kProfRow, 0, 0);
		sslm_launch::RowNormArgs a{st.codes, st.idx, H, m->layers[l0].attn_gain, m->layers[l0].attn_norm,
		                           m->normed, m->normed_scale, m->normed_recip};
		sslm_launch::rmsnorm(a, M, H, m->tok, m->status, l0, s);
		ck(hipGetLastError());
	}
	for (int l = l0; l < l1; ++l) {
		const DevLayer& lw = m->layers[l];
		RawIn raw{};  // the last projection's split-K partials, when it split
		// q | k | v projection (forward_sites.cpp:1699-1735)
		{
			const int pj[3] = {0, 1, 2};
			run_lora_u(m, ad, l, pj, 3, m->normed, M, H);
			GemmArgs g = gemm_args(m, m->normed, M, H, lw.w_qkv, H + 2 * KVH, H);
			g.epi.layer = l;
			g.epi.in_recip = m->normed_recip;
			g.epi.in_scale = m->normed_scale;
			g.epi.rank = ad ? (int)ad->rank : 0;
			g.epi.nseg = 3;
			g.epi.seg[0] = funnel_seg(0, H, m->q_f, H, m->mx_q, lw.f_qkv, lw.b_q);
			Segment sk{};
			sk.n_begin = H;
			sk.n_end = H + KVH;
			sk.mode = kSegWide;
			sk.out = m->kv_f;
			sk.ld_out = 2 * KVH;
			sk.fold = lw.f_qkv + 3 * H;
			sk.bias = lw.b_k;
			Segment sv = sk;
			sv.n_begin = H + KVH;
			sv.n_end = H + 2 * KVH;
			sv.out = m->kv_f + KVH;
			sv.fold = lw.f_qkv + 3 * (H + KVH);
			sv.bias = lw.b_v;
			g.epi.seg[1] = sk;
			g.epi.seg[2] = sv;
			attach_lora(m, ad, l, 0, &g.epi.seg[0], 0);
			attach_lora(m, ad, l, 1, &g.epi.seg[1], 1);
			attach_lora(m, ad, l, 2, &g.epi.seg[2], 2);
			raw = split_raw(m, g, H <= 4096);
			run_gemm(m, g, kProfGemm);
		}
		{
			sslm_launch::QkvPostArgs a{};
			a.M = M;
			a.H = H;
			a.NH = m->NH;
			a.NKV = m->NKV;
			a.D = m->D;
			a.cap = m->cap;
			a.tok = m->tok;
			a.q_f = m->q_f;
			a.q_maxpart = m->mx_q;
			a.kv_f = m->kv_f;
			a.in_scale = m->normed_scale;
			a.q_site = lw.q;
			a.r_t_k = lw.r_t_k;
			a.e_t_k = lw.e_t_k;
			a.r_t_v = lw.r_t_v;
			a.e_t_v = lw.e_t_v;
			a.rope_cos = m->rope_cos;
			a.rope_sin = m->rope_sin;
			a.block_bytes = (int64_t)m->block_bytes;
			a.layer = l;
			a.q_rot = m->q_rot;
			a.q_scale = m->q_scale;
			a.sat = m->sat;
			a.status = m->status;
			a.kv_pool = m->pool_dev;
			a.raw = raw;
			ProfScope p(s, kProfRow, 0, 0);
			sslm_launch::qkv_post(a, s);
			ck(hipGetLastError());
		}
		{
			sslm_launch::AttnArgs a{};
			a.M = M;
			a.H = H;
			a.NH = m->NH;
			a.NKV = m->NKV;
			a.D = m->D;
			a.cap = m->cap;
			a.tok = m->tok;
			a.q_rot = m->q_rot;
			a.q_scale = m->q_scale;
			a.khead_m = lw.khead_m;
			a.khead_e = lw.khead_e;
			a.ctx_fold = lw.ctx_fold;
			a.kv_pool = m->pool_dev;
			a.block_bytes = (int64_t)m->block_bytes;
			a.layer = l;
			a.ln2_q = m->ln2_q;
			a.b_q = m->b_q;
			a.ca_q = m->ca_q;
			a.ctx_f = m->ctx_f;
			a.ctx_maxpart = m->mx_ctx;
			a.scratch = m->attn_scratch;
			a.status = m->status;
			ProfScope p(s, kProfAttn, 0, 0);
			sslm_launch::attention(a, s);
			ck(hipGetLastError());
		}
		{
			sslm_launch::FunnelArgs a{};
			a.M = M;
			a.N = H;
			a.tok = m->tok;
			a.f = m->ctx_f;
			a.ld_f = H;
			a.maxpart = m->mx_ctx;
			a.ntiles = m->NH;
			a.incoming = nullptr;
			a.site = lw.ctx;
			a.out = m->ctx;
			a.out_scale = m->ctx_scale;
			a.layer = l;
			a.status = m->status;
			ProfScope p(s, kProfRow, 0, 0);
			sslm_launch::funnel(a, s);
			ck(hipGetLastError());
		}
		{  // o_proj (forward_sites.cpp:1907-1914)
			const int pj[1] = {3};
			run_lora_u(m, ad, l, pj, 1, m->ctx, M, H);
			GemmArgs g = gemm_args(m, m->ctx, M, H, lw.w_o, H, H);
			g.epi.layer = l;
			g.epi.rank = ad ? (int)ad->rank : 0;
			g.epi.nseg = 1;
			g.epi.seg[0] = funnel_seg(0, H, m->o_f, H, m->mx_o, lw.f_o, nullptr);
			attach_lora(m, ad, l, 3, &g.epi.seg[0], 0);
			raw = split_raw(m, g, H <= 6144);
			run_gemm(m, g, kProfGemm);
		}
		{  // attn residual -> mlp norm (forward_sites.cpp:1923-1936)
			sslm_launch::ResidualArgs a{};
			a.M = M;
			a.H = H;
			a.tok = m->tok;
			a.branch_f = m->o_f;
			a.branch_maxpart = m->mx_o;
			a.branch_in = m->ctx_scale;
			a.branch_site = lw.o;
			a.stream = st.codes;
			a.stream_idx = st.idx;
			a.stream_scale = st.scale;
			a.res_site = lw.attn_res;
			a.out_stream = m->attn_stream;
			a.out_idx = m->ident;
			a.out_stream_scale = m->attn_stream_scale;
			a.gain = lw.mlp_gain;
			a.norm_site = lw.mlp_norm;
			a.norm_out = m->mlp_normed;
			a.norm_scale = m->mlp_scale;
			a.norm_recip = m->mlp_recip;
			a.layer = l;
			a.status = m->status;
			a.raw = raw;
			ProfScope p(s, kProfRow, 0, 0);
			sslm_launch::residual_norm(a, s);
			ck(hipGetLastError());
		}
		{  // gate | up (forward_sites.cpp:1938-1955)
			const int pj[2] = {4, 5};
			run_lora_u(m, ad, l, pj, 2, m->mlp_normed, M, H);
			GemmArgs g = gemm_args(m, m->mlp_normed, M, H, lw.w_gu, 2 * I, H);
			g.epi.layer = l;
			g.epi.rank = ad ? (int)ad->rank : 0;
			g.epi.nseg = 2;
			g.epi.seg[0] = funnel_seg(0, I, m->gu_f, 2 * I, m->mx_gu, lw.f_gu, nullptr);
			g.epi.seg[1] = funnel_seg(I, 2 * I, m->gu_f + I, 2 * I, m->mx_gu, lw.f_gu + 3 * I, nullptr);
			attach_lora(m, ad, l, 4, &g.epi.seg[0], 0);
			attach_lora(m, ad, l, 5, &g.epi.seg[1], 1);
			raw = split_raw(m, g, I <= 4096);
			run_gemm(m, g, kProfGemm);
		}
		{
			sslm_launch::ActArgs a{};
			a.M = M;
			a.I = I;
			a.tok = m->tok;
			a.gu_f = m->gu_f;
			a.gu_maxpart = m->mx_gu;
			a.in_scale = m->mlp_scale;
			a.gate_site = lw.gate;
			a.up_site = lw.up;
			a.act_site = lw.act;
			a.silu = m->silu;
			a.act = m->act;
			a.act_scale = m->act_scale;
			a.layer = l;
			a.status = m->status;
			a.raw = raw;
			ProfScope p(s, kProfRow, 0, 0);
			sslm_launch::mlp_act(a, s);
			ck(hipGetLastError());
		}
		{  // down_proj (forward_sites.cpp:1969-1977)
			const int pj[1] = {6};
			run_lora_u(m, ad, l, pj, 1, m->act, M, I);
			GemmArgs g = gemm_args(m, m->act, M, I, lw.w_down, H, I);
			g.epi.layer = l;
			g.epi.rank = ad ? (int)ad->rank : 0;
			g.epi.nseg = 1;
			g.epi.seg[0] = funnel_seg(0, H, m->down_f, H, m->mx_down, lw.f_down, nullptr);
			attach_lora(m, ad, l, 6, &g.epi.seg[0], 0);
			raw = split_raw(m, g, H <= 6144);
			run_gemm(m, g, kProfGemm);
		}
		{  // mlp residual -> commit -> next layer's attn norm (forward_sites.cpp:1982-2009)
			sslm_launch::ResidualArgs a{};
			a.M = M;
			a.H = H;
			a.tok = m->tok;
			a.branch_f = m->down_f;
			a.branch_maxpart = m->mx_down;
			a.branch_in = m->act_scale;
			a.branch_site = lw.down;
			a.stream = m->attn_stream;
			a.stream_idx = m->ident;
			a.stream_scale = m->attn_stream_scale;
			a.res_site = lw.mlp_res;
			a.out_stream = st.codes;
			a.out_idx = st.idx;
			a.out_stream_scale = st.scale;
			if (l + 1 < l1) {
				a.gain = m->layers[l + 1].attn_gain;
				a.norm_site = m->layers[l + 1].attn_norm;
				a.norm_out = m->normed;
				a.norm_scale = m->normed_scale;
				a.norm_recip = m->normed_recip;
			}
			a.layer = l;
			a.status = m->status;
			a.raw = raw;
			ProfScope p(s, kProfRow, 0, 0);
			sslm_launch::residual_norm(a, s);
			ck(hipGetLastError());
		}
	}
}


// final norm + LM head + lowest-index argmax for M tokens whose stream rows are st.idx
// (src/sslm_abi.cpp:2280-2289, forward_sites.cpp:2412-2441)
void run_logits(sslm_model m, int M, StreamRef st) {
	hipStream_t s = m->stream;
	{
		ProfScope p(s, kProfRow, 0, 0);
		sslm_launch::RowNormArgs a{st.codes, st.idx, m->H, m->final_gain, m->final_site, m->final_codes,
		                           m->final_scale, nullptr};
		sslm_launch::rmsnorm(a, M, m->H, m->tok, m->status, m->L, s);
		ck(hipGetLastError());
	}
	GemmArgs g = gemm_args(m, m->final_codes, M, m->H, m->head, m->V, m->H);
	g.epi.argmax_key = m->argmax_key;
	g.epi.key_ld = (m->V + 15) / 16;
	g.epi.layer = m->L;
	run_gemm(m, g, kProfHead);
	sslm_launch::argmax_finalize(m->argmax_key, (m->V + 15) / 16, M, m->out_tokens, s);
	ck(hipGetLastError());
}

sslm_status map_forward_status(int32_t word) {
	const int32_t st = word & 0xff;
	if (st == 0) return SSLM_OK;
	if (st == kSoftmaxKernelRefusedAfterGateAccepted) return SSLM_NUMERIC_STEP_REFUSED;
	return SSLM_ARTIFACT_REJECTED;  // src/sslm_abi.cpp:1352-1360
}

template <typename F>
sslm_status guarded(F&& f) {
	try {
		return f();
	} catch (const HipError& e) {
		fprintf(stderr, "sslm_hip: HIP error %d (%s)\n", (int)e.e, hipGetErrorString(e.e));
		return e.e == hipErrorOutOfMemory ? SSLM_ALLOCATION_FAILED : SSLM_INVALID_ARGUMENT;
	} catch (const std::bad_alloc&) {
		return SSLM_ALLOCATION_FAILED;
	}
}

bool aligned64(const void* p) { return ((uintptr_t)p % SSLM_ABI_ALIGNMENT_BYTES) == 0; }

const TensorView* need(const std::map<std::string, TensorView>& m, const std::string& k, uint64_t elems,
                       std::string* err) {
	auto it = m.find(k);
	if (it == m.end()) {
		*err = "missing tensor " + k;
		return nullptr;
	}
	if (elems && it->second.elems != elems) {
		*err = "tensor " + k + " has the wrong size";
		return nullptr;
	}
	return &it->second;
}

bool read_scale(const Artifact& a, const std::string& k, Scale* out, std::string* err) {
	auto it = a.composition.find(k);
	if (it == a.composition.end()) {
		*err = "missing composition constant " + k;
		return false;
	}
	*out = Scale{it->second.v[0], it->second.v[1]};
	return true;
}

template <typename T>
void append_le(std::vector<T>* out, const TensorView& t) {
	const size_t n = t.elems;
	const size_t base = out->size();
	out->resize(base + n);
	memcpy(out->data() + base, t.data, n * sizeof(T));  // little-endian host
}

// Upload one model (layer_marshal.h:141-330 naming; src/sslm_abi.cpp:609-676 embed/head/final).
bool build_device_model(sslm_model m, std::string* err) {
	const Artifact& A = m->art;
	const ModelConfig& c = A.config;
	m->c = c;
	m->H = c.hidden;
	m->L = c.layers;
	m->NH = c.heads;
	m->NKV = c.kv_heads;
	m->D = c.head_dim;
	m->I = c.inter;
	m->V = c.vocab;
	m->KVH = m->NKV * m->D;
	m->cap = c.context_cap;
	m->block_bytes = (size_t)c.layers * c.context_cap * c.kv_heads * c.head_dim * 2 * (c.kv_precision ? 2 : 1);
	if (c.kv_precision != 0) {
		*err = "int16 KV precision has no decode path (forward_sites.cpp:2503)";
		return false;
	}
	if (m->H % 64 || m->I % 64 || m->KVH % 16 || m->NH % m->NKV ||
	    !sslm_launch::row_geometry_ok(m->H, m->I, m->NKV, m->D)) {
		*err = "geometry outside this backend's tiling (hidden, intermediate multiple of 64; hidden <= 8192; "
		       "intermediate <= 20480; head_dim 32, 64, 128 or 256; kv width <= 2048)";
		return false;
	}
	auto& own = m->owned;
	const int H = m->H, I = m->I, KVH = m->KVH;
	m->layers.resize(m->L);
	for (int l = 0; l < m->L; ++l) {
		const std::string p = "layer" + std::to_string(l) + ".";
		DevLayer& d = m->layers[l];
		std::vector<int8_t> w;
		std::vector<int32_t> f;
		const char* qkv[3] = {"q_proj", "k_proj", "v_proj"};
		const uint64_t rows[3] = {(uint64_t)H, (uint64_t)KVH, (uint64_t)KVH};
		for (int i = 0; i < 3; ++i) {
			const TensorView* t = need(A.weights, p + qkv[i], rows[i] * H, err);
			const TensorView* fs = need(A.weight_scales, p + qkv[i], rows[i] * 3, err);
			if (!t || !fs) return false;
			append_le(&w, *t);
			append_le(&f, *fs);
		}
		d.w_qkv = dupload(w, &own);
		d.f_qkv = dupload(f, &own);
		int64_t* biases[3] = {nullptr, nullptr, nullptr};
		for (int i = 0; i < 3; ++i) {
			auto it = A.biases.find(p + qkv[i]);
			if (it == A.biases.end()) continue;
			if (it->second.elems != rows[i]) {
				*err = "bias " + p + qkv[i] + " has the wrong size";
				return false;
			}
			std::vector<int64_t> b;
			append_le(&b, it->second);
			biases[i] = dupload(b, &own);
		}
		d.b_q = biases[0];
		d.b_k = biases[1];
		d.b_v = biases[2];
		auto up1 = [&](const char* name, uint64_t n, uint64_t k, int8_t** wd, int32_t** fd) -> bool {
			const TensorView* t = need(A.weights, p + name, n * k, err);
			const TensorView* fs = need(A.weight_scales, p + name, n * 3, err);
			if (!t || !fs) return false;
			std::vector<int8_t> ww;
			std::vector<int32_t> ff;
			append_le(&ww, *t);
			append_le(&ff, *fs);
			*wd = dupload(ww, &own);
			*fd = dupload(ff, &own);
			return true;
		};
		if (!up1("o_proj", H, H, &d.w_o, &d.f_o)) return false;
		if (!up1("down_proj", H, I, &d.w_down, &d.f_down)) return false;
		{
			std::vector<int8_t> ww;
			std::vector<int32_t> ff;
			for (const char* nm : {"gate_proj", "up_proj"}) {
				const TensorView* t = need(A.weights, p + nm, (uint64_t)I * H, err);
				const TensorView* fs = need(A.weight_scales, p + nm, (uint64_t)I * 3, err);
				if (!t || !fs) return false;
				append_le(&ww, *t);
				append_le(&ff, *fs);
			}
			d.w_gu = dupload(ww, &own);
			d.f_gu = dupload(ff, &own);
		}
		{
			const TensorView* t = need(A.weight_scales, p + "ctx_fold", (uint64_t)m->NH * 3, err);
			if (!t) return false;
			std::vector<int32_t> ff;
			append_le(&ff, *t);
			d.ctx_fold = dupload(ff, &own);
		}
		for (int i = 0; i < 2; ++i) {
			const TensorView* t = need(A.weights, p + (i ? "mlp_norm.gain" : "attn_norm.gain"), H, err);
			if (!t) return false;
			std::vector<int32_t> g(H);
			for (int k = 0; k < H; ++k) g[k] = (int32_t)(int8_t)t->data[k];  // layer_marshal.h:58-60
			(i ? d.mlp_gain : d.attn_gain) = dupload(g, &own);
		}
		std::vector<int64_t> rk(m->NKV), ek(m->NKV), rv(m->NKV), ev(m->NKV), km(m->NKV), ke(m->NKV);
		for (int h = 0; h < m->NKV; ++h) {
			auto kk = A.kv_landing_recip.find(p + "k_head" + std::to_string(h));
			auto vv = A.kv_landing_recip.find(p + "v_head" + std::to_string(h));
			auto sm = A.composition.find(p + "softmax_khead" + std::to_string(h));
			if (kk == A.kv_landing_recip.end() || vv == A.kv_landing_recip.end() || sm == A.composition.end()) {
				*err = p + ": missing kv landing / softmax_khead constants";
				return false;
			}
			ek[h] = kk->second.v[1];
			rk[h] = kk->second.v[2];
			ev[h] = vv->second.v[1];
			rv[h] = vv->second.v[2];
			km[h] = sm->second.v[0];
			ke[h] = sm->second.v[1];
		}
		d.r_t_k = dupload(rk, &own);
		d.e_t_k = dupload(ek, &own);
		d.r_t_v = dupload(rv, &own);
		d.e_t_v = dupload(ev, &own);
		d.khead_m = dupload(km, &own);
		d.khead_e = dupload(ke, &own);
		struct {
			const char* k;
			Scale* s;
		} sites[] = {{"attn_norm", &d.attn_norm}, {"q_proj", &d.q},       {"o_proj", &d.o},
		             {"attn_ctx", &d.ctx},        {"attn_residual", &d.attn_res}, {"mlp_norm", &d.mlp_norm},
		             {"gate_proj", &d.gate},      {"up_proj", &d.up},     {"mlp_act", &d.act},
		             {"down_proj", &d.down},      {"mlp_residual", &d.mlp_res}};
		for (auto& st : sites)
			if (!read_scale(A, p + st.k, st.s, err)) return false;
	}
	{
		const TensorView* e = need(A.weights, "embed", (uint64_t)m->V * H, err);
		const TensorView* g = need(A.weights, "final_norm.gain", H, err);
		if (!e || !g) return false;
		std::vector<int8_t> ew;
		append_le(&ew, *e);
		m->embed = dupload(ew, &own);
		if (c.tie_embeddings) {
			m->head = m->embed;
		} else {
			const TensorView* h = need(A.weights, "lm_head", (uint64_t)m->V * H, err);
			if (!h) {
				*err = "tie_word_embeddings=0 but no lm_head tensor";
				return false;
			}
			std::vector<int8_t> hw;
			append_le(&hw, *h);
			m->head = dupload(hw, &own);
		}
		std::vector<int32_t> fg(H);
		for (int k = 0; k < H; ++k) fg[k] = (int32_t)(int8_t)g->data[k];
		m->final_gain = dupload(fg, &own);
		if (!read_scale(A, "embed", &m->embed_site, err) || !read_scale(A, "final_norm", &m->final_site, err))
			return false;
	}
	{
		const TensorView* cs = need(A.rope, "cos", (uint64_t)m->cap * (m->D / 2), err);
		const TensorView* sn = need(A.rope, "sin", (uint64_t)m->cap * (m->D / 2), err);
		if (!cs || !sn) return false;
		std::vector<int64_t> cv, sv;
		append_le(&cv, *cs);
		append_le(&sv, *sn);
		m->rope_cos = dupload(cv, &own);
		m->rope_sin = dupload(sv, &own);
		m->silu = dupload(A.sigmoid_lut, &own);
	}
	{  // include/superslm/intmath.h:518-527 -- truncations of the same doubles
		const double ln2 = 0x1.62e42fefa39efp-1;
		m->ln2_q = (int64_t)(ln2 * (double)((int64_t)1 << 30));
		m->b_q = (int64_t)(1.353 * (double)((int64_t)1 << 30));
		m->ca_q = (int64_t)((0.344 / 0.3585) * (double)((int64_t)1 << 30));
	}
	// slots
	m->stream_codes = dalloc<int8_t>((size_t)kSlotCapacity * H, &own);
	m->stream_scale = dalloc<Scale>(kSlotCapacity, &own);
	m->sat = dalloc<unsigned long long>(kSlotCapacity, &own);
	m->status = dalloc<int32_t>(kSlotCapacity, &own);
	for (int i = kSlotCapacity - 1; i >= 0; --i) m->free_slots.push_back(i);
	// workspace
	const int T = kMaxTokens;
	m->tok = dalloc<TokenInfo>(T, &own);
	m->tok_ids = dalloc<int32_t>(T, &own);
	m->ident = dalloc<int32_t>(T, &own);
	{
		std::vector<int32_t> id(T);
		for (int i = 0; i < T; ++i) id[i] = i;
		ck(hipMemcpy(m->ident, id.data(), T * 4, hipMemcpyHostToDevice));
	}
	m->slot_idx = dalloc<int32_t>(T, &own);
	m->out_tokens = dalloc<int32_t>(T, &own);
	m->hid_chunk = dalloc<int8_t>((size_t)T * H, &own);
	m->normed = dalloc<int8_t>((size_t)T * H, &own);
	m->q_rot = dalloc<int8_t>((size_t)T * H, &own);
	m->ctx = dalloc<int8_t>((size_t)T * H, &own);
	m->attn_stream = dalloc<int8_t>((size_t)T * H, &own);
	m->mlp_normed = dalloc<int8_t>((size_t)T * H, &own);
	m->act = dalloc<int8_t>((size_t)T * I, &own);
	m->final_codes = dalloc<int8_t>((size_t)T * H, &own);
	for (Scale** sp : {&m->hid_chunk_scale, &m->normed_scale, &m->q_scale, &m->ctx_scale, &m->attn_stream_scale,
	                   &m->mlp_scale, &m->act_scale, &m->final_scale})
		*sp = dalloc<Scale>(T, &own);
	m->normed_recip = dalloc<int64_t>(T, &own);
	m->mlp_recip = dalloc<int64_t>(T, &own);
	m->kv_f = dalloc<int64_t>((size_t)T * 2 * KVH, &own);
	m->q_f = dalloc<int32_t>((size_t)T * H, &own);
	m->ctx_f = dalloc<int32_t>((size_t)T * H, &own);
	m->o_f = dalloc<int32_t>((size_t)T * H, &own);
	m->gu_f = dalloc<int32_t>((size_t)T * 2 * I, &own);
	m->down_f = dalloc<int32_t>((size_t)T * H, &own);
	m->mx_q = dalloc<uint32_t>((size_t)(H + 2 * KVH) / 16 * kPartLd, &own);
	m->mx_ctx = dalloc<uint32_t>((size_t)m->NH * kPartLd, &own);
	m->mx_o = dalloc<uint32_t>((size_t)H / 16 * kPartLd, &own);
	m->mx_gu = dalloc<uint32_t>((size_t)2 * I / 16 * kPartLd, &own);
	m->mx_down = dalloc<uint32_t>((size_t)H / 16 * kPartLd, &own);
	m->argmax_key = dalloc<unsigned long long>((size_t)(m->V + 15) / 16 * kPartLd, &own);
	{
		const int shapes[4][2] = {{H + 2 * KVH, H}, {H, H}, {2 * I, H}, {H, I}};
		size_t elems = 0;
		for (auto& sh : shapes) {
			if (sslm_launch::gemv_eligible(64, sh[1]))
				elems = std::max(elems, (size_t)sslm_launch::gemv_plan(64, sh[0], sh[1], true).splits * 64 * sh[0]);
			for (int rows = 65; rows <= kMaxTokens; ++rows) {
				const int sp = sslm_launch::prefill_plan(rows, sh[0], sh[1], true).splits;
				if (sp > 1) elems = std::max(elems, (size_t)sp * rows * sh[0]);
			}
		}
		m->raw_part = elems ? dalloc<int32_t>(elems, &own) : nullptr;
	}
	for (int i = 0; i < 3; ++i) m->lora_u[i] = dalloc<int8_t>((size_t)T * kMaxRank, &own);
	if (!sslm_launch::attention_in_lds(m->cap))
		m->attn_scratch = dalloc<int64_t>((size_t)T * m->NH * m->cap, &own);
	else
		m->attn_scratch = nullptr;
	ck(hipStreamCreate(&m->stream));
	return true;
}

void free_model(sslm_model m) {
	if (m->stream) (void)hipStreamSynchronize(m->stream);
	for (void* p : m->owned) (void)hipFree(p);
	m->owned.clear();
	if (m->stream) (void)hipStreamDestroy(m->stream);
	m->stream = nullptr;
}

// Upload the TokenInfo of one launch sequence.
void put_tokens(sslm_model m, const std::vector<TokenInfo>& ti) {
	ck(hipMemcpyAsync(m->tok, ti.data(), ti.size() * sizeof(TokenInfo), hipMemcpyHostToDevice, m->stream));
}

// prefill of `n` admitted tokens (PrefillWholeTokensImpl, src/sslm_abi.cpp:1481-1535)
sslm_status prefill_tokens(sslm_model m, sslm_seq s, const int32_t* tokens, int n) {
	m->pool_dev = s->pool->dev;
	const int H = m->H;
	int done = 0;
	while (done < n) {
		const int T = std::min(kMaxTokens, n - done);
		std::vector<TokenInfo> ti(T);
		for (int t = 0; t < T; ++t) ti[t] = TokenInfo{s->context_length + done + t, s->slot, (int32_t)s->block};
		put_tokens(m, ti);
		ck(hipMemcpyAsync(m->tok_ids, tokens + done, T * 4, hipMemcpyHostToDevice, m->stream));
		{
			ProfScope p(m->stream, kProfRow, 0, 0);
			sslm_launch::embed(m->tok_ids, T, m->embed, H, m->V, m->embed_site, m->hid_chunk, m->ident,
			                   m->hid_chunk_scale, m->ident, m->tok, m->status, m->stream);
			ck(hipGetLastError());
		}
		run_layers(m, T, StreamRef{m->hid_chunk, m->hid_chunk_scale, m->ident}, 0, m->L, s->adapter);
		int32_t word = 0;
		ck(hipMemcpyAsync(&word, m->status + s->slot, 4, hipMemcpyDeviceToHost, m->stream));
		ck(hipStreamSynchronize(m->stream));
		prof_collect();
		if (word != 0) {
			ck(hipMemset(m->status + s->slot, 0, 4));
			return map_forward_status(word);
		}
		// the chunk's last row becomes the sequence's stream state
		ck(hipMemcpyAsync(m->stream_codes + (size_t)s->slot * H, m->hid_chunk + (size_t)(T - 1) * H, H,
		                  hipMemcpyDeviceToDevice, m->stream));
		ck(hipMemcpyAsync(m->stream_scale + s->slot, m->hid_chunk_scale + (T - 1), sizeof(Scale),
		                  hipMemcpyDeviceToDevice, m->stream));
		s->context_length += T;
		s->layer_index = 0;
		done += T;
	}
	ck(hipStreamSynchronize(m->stream));
	return SSLM_OK;
}

}  // namespace

// ==========================================================================================
// C ABI
// ==========================================================================================
extern "C" {

sslm_status sslm_model_map(const void* data, size_t size, sslm_model* out) {
	if (!out) return SSLM_INVALID_ARGUMENT;
	*out = nullptr;
	if (!data) return SSLM_INVALID_ARGUMENT;
	return guarded([&]() -> sslm_status {
		std::unique_ptr<sslm_model_s> m(new sslm_model_s());
		std::string err;
		if (!parse_artifact((const uint8_t*)data, size, &m->art, &err)) {
			fprintf(stderr, "sslm_hip: artifact rejected: %s\n", err.c_str());
			return SSLM_ARTIFACT_REJECTED;
		}
		bool ok = false;
		try {
			ok = build_device_model(m.get(), &err);
		} catch (...) {
			free_model(m.get());
			throw;
		}
		if (!ok) {
			fprintf(stderr, "sslm_hip: artifact rejected: %s\n", err.c_str());
			free_model(m.get());
			return SSLM_ARTIFACT_REJECTED;
		}
		*out = m.release();
		return SSLM_OK;
	});
}

sslm_status sslm_model_unmap(sslm_model model) {
	if (!model) return SSLM_INVALID_ARGUMENT;
	if (model->live_refs.load() != 0) return SSLM_MODEL_HAS_LIVE_SEQUENCES;
	free_model(model);
	delete model;
	return SSLM_OK;
}

size_t sslm_kv_block_size(sslm_model model) { return model ? model->block_bytes : 0; }

size_t sslm_kv_pool_overhead_size(sslm_model model, uint32_t block_count) {
	if (!model) return 0;
	return (size_t)block_count * sizeof(uint32_t) * 2 + 32;  // src/sslm_abi.cpp:870-877
}

size_t sslm_seq_state_size(sslm_model model) {
	if (!model) return 0;  // src/sslm_abi.cpp:879-890
	return 124 + (size_t)model->H + (size_t)model->cap * 4 + model->block_bytes;
}

sslm_status sslm_kv_pool_create(sslm_model model, void* buf, size_t buf_size, uint32_t block_count,
                                sslm_kv_pool* out) {
	if (!out) return SSLM_INVALID_ARGUMENT;
	*out = nullptr;
	if (!model || !buf || block_count == 0) return SSLM_INVALID_ARGUMENT;
	const size_t bs = model->block_bytes;
	if (bs == 0 || (size_t)block_count > SIZE_MAX / bs) return SSLM_INVALID_ARGUMENT;
	const size_t required = (size_t)block_count * bs + sslm_kv_pool_overhead_size(model, block_count);
	if (buf_size < required) return SSLM_BUFFER_TOO_SMALL;
	if (!aligned64(buf)) return SSLM_MISALIGNED_BUFFER;
	return guarded([&]() -> sslm_status {
		std::unique_ptr<sslm_kv_pool_s> p(new sslm_kv_pool_s());
		p->model = model;
		p->buf = buf;
		p->buf_size = buf_size;
		p->block_count = block_count;
		p->block_size = bs;
		void* d = nullptr;
		ck(hipMalloc(&d, (size_t)block_count * bs));
		p->dev = (int8_t*)d;
		for (uint32_t i = 0; i < block_count; ++i) p->free_list.push_back(i);
		model->live_refs++;
		*out = p.release();
		return SSLM_OK;
	});
}

sslm_status sslm_kv_pool_destroy(sslm_kv_pool pool) {
	if (!pool) return SSLM_INVALID_ARGUMENT;
	if (pool->live_refs.load() != 0) return SSLM_POOL_HAS_LIVE_HANDLES;
	(void)hipStreamSynchronize(pool->model->stream);
	(void)hipFree(pool->dev);
	pool->model->live_refs--;
	delete pool;
	return SSLM_OK;
}

size_t sslm_workspace_size(sslm_model model, const sslm_config* config) {
	if (!model || !config) return 0;
	if (config->max_batch < 1 || config->max_chunk_budget < 1 || config->max_layer_budget < 1 ||
	    config->max_layer_budget > model->L || config->reserved != 0)
		return 0;
	// host-side per-call bookkeeping: one status and token slot per batch entry
	return 64 + (size_t)config->max_batch * 16 + (size_t)config->max_chunk_budget * 4;
}

sslm_status sslm_workspace_create(sslm_model model, const sslm_config* config, void* buf, size_t buf_size,
                                  sslm_workspace* out) {
	if (!out) return SSLM_INVALID_ARGUMENT;
	*out = nullptr;
	const size_t req = sslm_workspace_size(model, config);
	if (!req || !buf) return SSLM_INVALID_ARGUMENT;
	if (buf_size < req) return SSLM_BUFFER_TOO_SMALL;
	if (!aligned64(buf)) return SSLM_MISALIGNED_BUFFER;
	sslm_workspace_s* w = new (std::nothrow) sslm_workspace_s();
	if (!w) return SSLM_ALLOCATION_FAILED;
	w->buf = buf;
	w->buf_size = buf_size;
	w->config = *config;
	memset(buf, 0, req);
	*out = w;
	return SSLM_OK;
}

sslm_status sslm_workspace_destroy(sslm_workspace ws) {
	if (!ws) return SSLM_INVALID_ARGUMENT;
	delete ws;
	return SSLM_OK;
}

sslm_status sslm_seq_create(sslm_model model, sslm_kv_pool* pool, sslm_seq* out) {
	if (!out) return SSLM_INVALID_ARGUMENT;
	*out = nullptr;
	if (!model || !pool || !*pool) return SSLM_INVALID_ARGUMENT;
	sslm_kv_pool p = *pool;
	if (p->model != model) return SSLM_INVALID_ARGUMENT;
	return guarded([&]() -> sslm_status {
		std::lock_guard<std::mutex> lk(model->mu);
		uint32_t block;
		{
			std::lock_guard<std::mutex> pl(p->mu);
			if (p->free_list.empty()) return SSLM_KV_POOL_EXHAUSTED;
			if (model->free_slots.empty()) return SSLM_ALLOCATION_FAILED;
			block = p->free_list.back();  // src/sslm_abi.cpp:1308-1331: the list's back first
			p->free_list.pop_back();
			p->live_refs++;
		}
		const int slot = model->free_slots.back();
		model->free_slots.pop_back();
		ck(hipMemsetAsync(p->dev + (size_t)block * p->block_size, 0, p->block_size, model->stream));
		ck(hipMemsetAsync(model->stream_codes + (size_t)slot * model->H, 0, model->H, model->stream));
		ck(hipMemsetAsync(model->stream_scale + slot, 0, sizeof(Scale), model->stream));
		ck(hipMemsetAsync(model->sat + slot, 0, 8, model->stream));
		ck(hipMemsetAsync(model->status + slot, 0, 4, model->stream));
		ck(hipStreamSynchronize(model->stream));
		sslm_seq_s* s = new sslm_seq_s();
		s->model = model;
		s->pool = p;
		s->block = block;
		s->slot = slot;
		model->live_refs++;
		{
			std::lock_guard<std::mutex> rl(g_registry_mu);
			g_live_seqs.insert(s);
		}
		*out = s;
		return SSLM_OK;
	});
}

sslm_status sslm_seq_release(sslm_seq seq) {
	if (!seq) return SSLM_INVALID_ARGUMENT;
	{
		std::lock_guard<std::mutex> rl(g_registry_mu);
		if (!g_live_seqs.erase(seq)) return SSLM_INVALID_ARGUMENT;
	}
	sslm_model m = seq->model;
	{
		std::lock_guard<std::mutex> lk(m->mu);
		if (seq->adapter) seq->adapter->live_refs--;
		{
			std::lock_guard<std::mutex> pl(seq->pool->mu);
			seq->pool->free_list.push_back(seq->block);
			seq->pool->live_refs--;
		}
		m->free_slots.push_back(seq->slot);
		m->live_refs--;
	}
	delete seq;
	return SSLM_OK;
}

sslm_status sslm_seq_reset(sslm_seq seq) {
	if (!seq) return SSLM_INVALID_ARGUMENT;
	if (seq->layer_index != 0) return SSLM_SEQ_RESET_MIDTOKEN_REJECTED;  // src/sslm_abi.cpp:1820-1846
	sslm_model m = seq->model;
	return guarded([&]() -> sslm_status {
		std::lock_guard<std::mutex> lk(m->mu);
		ck(hipMemsetAsync(seq->pool->dev + (size_t)seq->block * seq->pool->block_size, 0, seq->pool->block_size,
		                  m->stream));
		ck(hipMemsetAsync(m->stream_codes + (size_t)seq->slot * m->H, 0, m->H, m->stream));
		ck(hipMemsetAsync(m->stream_scale + seq->slot, 0, sizeof(Scale), m->stream));
		ck(hipMemsetAsync(m->sat + seq->slot, 0, 8, m->stream));
		ck(hipStreamSynchronize(m->stream));
		seq->context_length = 0;
		seq->layer_index = 0;
		seq->current_token = -1;
		seq->ready_for_logits = false;
		return SSLM_OK;
	});
}

sslm_status sslm_prefill(sslm_model model, sslm_seq seq, const int32_t* tokens, int32_t count, int32_t chunk_budget,
                         sslm_span_kind kind, sslm_workspace ws, int32_t* consumed) {
	(void)ws;
	if (!consumed) return SSLM_INVALID_ARGUMENT;
	*consumed = 0;
	if (!model || !seq) return SSLM_INVALID_ARGUMENT;
	if (count < 0 || chunk_budget < 1 || (count > 0 && !tokens)) return SSLM_INVALID_ARGUMENT;
	if (kind == SSLM_SPAN_SCHEMA_CONTENT) return SSLM_SCHEMA_SPAN_UNBOUND;  // no schema can be bound
	if (seq->model != model) return SSLM_INVALID_ARGUMENT;
	return guarded([&]() -> sslm_status {
		std::lock_guard<std::mutex> lk(model->mu);
		std::lock_guard<std::mutex> sl(seq->mu);
		const int32_t n = std::min(count, chunk_budget);
		if (n == 0) return SSLM_OK;
		// admission (src/sslm_abi.cpp:1451-1480)
		int32_t admit_id = n;
		for (int32_t i = 0; i < n; ++i)
			if (tokens[i] < 0 || (uint32_t)tokens[i] >= (uint32_t)model->V) {
				admit_id = i;
				break;
			}
		const int64_t head = model->cap - seq->context_length;
		const int32_t admit_cap = head <= 0 ? 0 : (head >= n ? n : (int32_t)head);
		const int32_t admit = std::min(admit_id, admit_cap);
		sslm_status stop = SSLM_OK;
		if (admit < n) stop = admit_id <= admit_cap ? SSLM_TOKEN_ID_OUT_OF_RANGE : SSLM_CONTEXT_CAP_EXCEEDED;
		if (admit > 0) {
			const sslm_status st = prefill_tokens(model, seq, tokens, admit);
			if (st != SSLM_OK) return st;
			seq->current_token = tokens[admit - 1];
			*consumed = admit;
			seq->ready_for_logits = true;  // src/sslm_abi.cpp:1969-1972
		}
		return stop;
	});
}

static sslm_status decode_batch(sslm_model m, sslm_seq* seqs, int32_t n, uint32_t budget, int32_t* out_tokens,
                                bool* stop_cap) {
	// Partition: sequences needing layers, grouped by their current layer; sequences needing logits.
	std::vector<int> need_logits;
	std::vector<std::pair<uint32_t, std::vector<int>>> groups;
	std::vector<int> embed_list;
	for (int i = 0; i < n; ++i) {
		sslm_seq s = seqs[i];
		if (s->ready_for_logits) {
			need_logits.push_back(i);
			continue;
		}
		if (s->layer_index == 0) {
			if (s->context_length >= m->cap) {  // src/sslm_abi.cpp:2233-2236
				*stop_cap = true;
				out_tokens[i] = -1;
				n = i;
				break;
			}
			embed_list.push_back(i);
		}
		auto it = std::find_if(groups.begin(), groups.end(), [&](auto& g) { return g.first == s->layer_index; });
		if (it == groups.end()) groups.push_back({s->layer_index, {i}});
		else it->second.push_back(i);
	}
	// drop group members past a cap stop
	for (auto& g : groups) g.second.erase(std::remove_if(g.second.begin(), g.second.end(), [&](int i) { return i >= n; }), g.second.end());
	need_logits.erase(std::remove_if(need_logits.begin(), need_logits.end(), [&](int i) { return i >= n; }), need_logits.end());
	embed_list.erase(std::remove_if(embed_list.begin(), embed_list.end(), [&](int i) { return i >= n; }), embed_list.end());

	// embeds (src/sslm_abi.cpp:2237-2249)
	for (size_t b = 0; b < embed_list.size(); b += kMaxTokens) {
		const int M = (int)std::min(embed_list.size() - b, (size_t)kMaxTokens);
		std::vector<TokenInfo> ti(M);
		std::vector<int32_t> ids(M), slots(M);
		for (int t = 0; t < M; ++t) {
			sslm_seq s = seqs[embed_list[b + t]];
			ti[t] = TokenInfo{s->context_length, s->slot, (int32_t)s->block};
			ids[t] = s->current_token;
			slots[t] = s->slot;
		}
		put_tokens(m, ti);
		ck(hipMemcpyAsync(m->tok_ids, ids.data(), M * 4, hipMemcpyHostToDevice, m->stream));
		ck(hipMemcpyAsync(m->slot_idx, slots.data(), M * 4, hipMemcpyHostToDevice, m->stream));
		ProfScope p(m->stream, kProfRow, 0, 0);
		sslm_launch::embed(m->tok_ids, M, m->embed, m->H, m->V, m->embed_site, m->stream_codes, m->slot_idx,
		                   m->stream_scale, m->slot_idx, m->tok, m->status, m->stream);
		ck(hipGetLastError());
		ck(hipStreamSynchronize(m->stream));  // slot_idx and tok are reused below
	}
	// layers, per group and per adapter
	std::vector<int> finished;
	for (auto& g : groups) {
		const uint32_t l0 = g.first;
		const uint32_t l1 = std::min<uint32_t>(m->L, l0 + budget);
		// one launch sequence per (adapter) partition of <= kMaxTokens tokens
		std::vector<sslm_adapter> ads;
		for (int i : g.second)
			if (std::find(ads.begin(), ads.end(), seqs[i]->adapter) == ads.end()) ads.push_back(seqs[i]->adapter);
		for (sslm_adapter ad : ads) {
			std::vector<int> members;
			for (int i : g.second)
				if (seqs[i]->adapter == ad) members.push_back(i);
			for (size_t b = 0; b < members.size(); b += kMaxTokens) {
				const int M = (int)std::min(members.size() - b, (size_t)kMaxTokens);
				std::vector<TokenInfo> ti(M);
				std::vector<int32_t> slots(M);
				for (int t = 0; t < M; ++t) {
					sslm_seq s = seqs[members[b + t]];
					ti[t] = TokenInfo{s->context_length, s->slot, (int32_t)s->block};
					slots[t] = s->slot;
				}
				// every sequence of one call shares the pool of the first (checked by the caller)
				m->pool_dev = seqs[members[b]]->pool->dev;
				put_tokens(m, ti);
				ck(hipMemcpyAsync(m->slot_idx, slots.data(), M * 4, hipMemcpyHostToDevice, m->stream));
				run_layers(m, M, StreamRef{m->stream_codes, m->stream_scale, m->slot_idx}, (int)l0, (int)l1, ad);
				ck(hipStreamSynchronize(m->stream));
			}
		}
		for (int i : g.second) {
			seqs[i]->layer_index = l1;
			if (l1 == (uint32_t)m->L) finished.push_back(i);
		}
	}
	// status check: a failure leaves its sequence at the failing layer (its last commit); every
	// other sequence of the batch advances normally
	std::vector<int32_t> words(kSlotCapacity);
	ck(hipMemcpy(words.data(), m->status, kSlotCapacity * 4, hipMemcpyDeviceToHost));
	prof_collect();
	sslm_status first_err = SSLM_OK;
	for (int i = 0; i < n; ++i) {
		sslm_seq s = seqs[i];
		const int32_t w = words[s->slot];
		if (w == 0) continue;
		s->layer_index = (uint32_t)std::min(w >> 8, m->L);
		ck(hipMemset(m->status + s->slot, 0, 4));
		if (first_err == SSLM_OK) first_err = map_forward_status(w);
		finished.erase(std::remove(finished.begin(), finished.end(), i), finished.end());
		need_logits.erase(std::remove(need_logits.begin(), need_logits.end(), i), need_logits.end());
		out_tokens[i] = -1;
	}
	for (int i : finished) seqs[i]->context_length += 1;
	for (auto& g : groups)
		for (int i : g.second)
			if (seqs[i]->layer_index < (uint32_t)m->L) out_tokens[i] = -1;
	// logits
	std::vector<int> lg = need_logits;
	lg.insert(lg.end(), finished.begin(), finished.end());
	for (size_t b = 0; b < lg.size(); b += kMaxTokens) {
		const int M = (int)std::min(lg.size() - b, (size_t)kMaxTokens);
		std::vector<TokenInfo> ti(M);
		std::vector<int32_t> slots(M);
		for (int t = 0; t < M; ++t) {
			sslm_seq s = seqs[lg[b + t]];
			ti[t] = TokenInfo{s->context_length, s->slot, (int32_t)s->block};
			slots[t] = s->slot;
		}
		put_tokens(m, ti);
		ck(hipMemcpyAsync(m->slot_idx, slots.data(), M * 4, hipMemcpyHostToDevice, m->stream));
		run_logits(m, M, StreamRef{m->stream_codes, m->stream_scale, m->slot_idx});
		std::vector<int32_t> toks(M);
		ck(hipMemcpyAsync(toks.data(), m->out_tokens, M * 4, hipMemcpyDeviceToHost, m->stream));
		ck(hipStreamSynchronize(m->stream));
		for (int t = 0; t < M; ++t) {
			sslm_seq s = seqs[lg[b + t]];
			s->ready_for_logits = false;
			s->current_token = toks[t];
			s->layer_index = 0;
			out_tokens[lg[b + t]] = toks[t];
		}
	}
	ck(hipMemcpy(words.data(), m->status, kSlotCapacity * 4, hipMemcpyDeviceToHost));
	prof_collect();
	for (int i : lg) {
		const int32_t w = words[seqs[i]->slot];
		if (w != 0) {
			ck(hipMemset(m->status + seqs[i]->slot, 0, 4));
			out_tokens[i] = -1;
			if (first_err == SSLM_OK) first_err = map_forward_status(w);
		}
	}
	return first_err;
}

static sslm_status decode_impl(sslm_model model, sslm_seq* seqs, int32_t n, const sslm_decode_params* params,
                               int32_t* out_tokens) {
	if (!model || !seqs || !params || !out_tokens) return SSLM_INVALID_ARGUMENT;
	if (n < 1) return SSLM_INVALID_ARGUMENT;
	if (params->struct_size != sizeof(sslm_decode_params)) return SSLM_INVALID_ARGUMENT;
	if (params->layer_budget < 1 || params->layer_budget > model->L) return SSLM_INVALID_ARGUMENT;
	if (params->mode != SSLM_DECODE_MODE_GREEDY) return SSLM_INVALID_ARGUMENT;
	for (int32_t i = 0; i < n; ++i)
		if (!seqs[i]) return SSLM_INVALID_ARGUMENT;
	return guarded([&]() -> sslm_status {
		std::lock_guard<std::mutex> lk(model->mu);
		std::vector<char> live(n, 0);
		{
			std::lock_guard<std::mutex> rl(g_registry_mu);
			for (int i = 0; i < n; ++i) live[i] = g_live_seqs.count(seqs[i]) ? 1 : 0;
		}
		for (int i = 0; i < n; ++i) {
			if (!live[i]) continue;
			if (seqs[i]->model != model) return SSLM_INVALID_ARGUMENT;
			if (seqs[i]->layer_index == 0 && seqs[i]->current_token < 0 && !seqs[i]->ready_for_logits)
				return SSLM_INVALID_ARGUMENT;
		}
		// batch runs of live, distinct sequences sharing one pool, in call order
		int i = 0;
		while (i < n) {
			if (!live[i]) {
				out_tokens[i] = -3;
				++i;
				continue;
			}
			std::vector<sslm_seq> run;
			std::vector<int> idx;
			std::set<sslm_seq> seen;
			int j = i;
			while (j < n && live[j] && !seen.count(seqs[j]) && seqs[j]->pool == seqs[i]->pool) {
				seen.insert(seqs[j]);
				run.push_back(seqs[j]);
				idx.push_back(j);
				++j;
			}
			std::vector<int32_t> out(run.size(), -1);
			bool stop_cap = false;
			const sslm_status st = decode_batch(model, run.data(), (int32_t)run.size(), (uint32_t)params->layer_budget,
			                                    out.data(), &stop_cap);
			for (size_t k = 0; k < run.size(); ++k) out_tokens[idx[k]] = out[k];
			if (st != SSLM_OK) return st;
			if (stop_cap) return SSLM_CONTEXT_CAP_EXCEEDED;
			i = j;
		}
		return SSLM_OK;
	});
}

sslm_status sslm_decode_step(sslm_model model, sslm_seq* seqs, int32_t n, const sslm_decode_params* params,
                             sslm_workspace ws, int32_t* out_tokens) {
	(void)ws;
	return decode_impl(model, seqs, n, params, out_tokens);
}

sslm_status sslm_decode_step_v2(sslm_model model, sslm_seq* seqs, int32_t n, const sslm_decode_params* params,
                                sslm_workspace ws, int32_t* out_tokens) {
	(void)ws;
	return decode_impl(model, seqs, n, params, out_tokens);
}

sslm_status sslm_decode_params_init(sslm_model model, int32_t mode, int32_t layer_budget, sslm_decode_params* out) {
	if (!model || !out || layer_budget < 1 || layer_budget > model->L) return SSLM_INVALID_ARGUMENT;
	if (mode != SSLM_DECODE_MODE_GREEDY && mode != SSLM_DECODE_MODE_DAMPED_GREEDY) return SSLM_INVALID_ARGUMENT;
	if (mode == SSLM_DECODE_MODE_DAMPED_GREEDY) return SSLM_ARTIFACT_REJECTED;  // no damped-greedy constants
	sslm_decode_params p{};
	p.layer_budget = layer_budget;
	p.struct_size = sizeof(p);
	p.mode = mode;
	*out = p;
	return SSLM_OK;
}

sslm_status sslm_stats(sslm_model model, sslm_seq seq, sslm_stats_out* out) {
	if (!model || !seq || !out) return SSLM_INVALID_ARGUMENT;
	memset(out, 0, sizeof(*out));
	out->kv_blocks_resident = 1;
	return SSLM_OK;
}

sslm_status sslm_g5_test_only_peek_kv_block_bytes(sslm_kv_pool pool, uint32_t block_index, uint8_t* out_buf,
                                                  size_t n) {
	if (!pool || !out_buf) return SSLM_INVALID_ARGUMENT;
	if (block_index >= pool->block_count || n > pool->block_size) return SSLM_INVALID_ARGUMENT;
	return guarded([&]() -> sslm_status {
		std::lock_guard<std::mutex> lk(pool->model->mu);
		ck(hipStreamSynchronize(pool->model->stream));
		ck(hipMemcpy(out_buf, pool->dev + (size_t)block_index * pool->block_size, n, hipMemcpyDeviceToHost));
		return SSLM_OK;
	});
}

sslm_status sslm_seq_save(sslm_seq seq, void* buf, size_t* n) {
	(void)seq;
	(void)buf;
	if (n) *n = 0;
	return SSLM_INVALID_ARGUMENT;
}

sslm_status sslm_adapter_map(const void* data, size_t size, sslm_model base, sslm_adapter* out) {
	(void)data;
	(void)size;
	(void)base;
	if (out) *out = nullptr;
	return SSLM_INVALID_ARGUMENT;
}

sslm_status sslm_adapter_release(sslm_adapter adapter) { return adapter ? SSLM_OK : SSLM_INVALID_ARGUMENT; }

size_t sslm_adapter_residency(sslm_adapter adapter) { return adapter ? adapter->bytes : 0; }

sslm_status sslm_seq_set_adapter(sslm_seq seq, sslm_adapter adapter) {
	if (!seq) return SSLM_INVALID_ARGUMENT;
	if (seq->layer_index != 0) return SSLM_ADAPTER_SWAP_MIDTOKEN_REJECTED;
	if (adapter && adapter->model != seq->model) return SSLM_ADAPTER_MODEL_MISMATCH;
	if (seq->adapter) seq->adapter->live_refs--;
	seq->adapter = adapter;
	if (adapter) adapter->live_refs++;
	return SSLM_OK;
}

// ---- outside the integer forward path ----
sslm_status sslm_prefix_begin(sslm_model, sslm_kv_pool*, sslm_prefix* out) {
	if (out) *out = nullptr;
	return SSLM_INVALID_ARGUMENT;
}
sslm_status sslm_prefix_prefill(sslm_model, sslm_prefix, const int32_t*, int32_t, int32_t, sslm_span_kind,
                                sslm_workspace, int32_t* consumed) {
	if (consumed) *consumed = 0;
	return SSLM_INVALID_ARGUMENT;
}
sslm_status sslm_prefix_freeze(sslm_prefix) { return SSLM_INVALID_ARGUMENT; }
sslm_status sslm_prefix_release(sslm_prefix) { return SSLM_INVALID_ARGUMENT; }
sslm_status sslm_seq_adopt_prefix(sslm_seq, sslm_prefix) { return SSLM_INVALID_ARGUMENT; }
sslm_status sslm_seq_restore(sslm_model, sslm_kv_pool*, const void*, size_t, sslm_seq* out) {
	if (out) *out = nullptr;
	return SSLM_INVALID_ARGUMENT;
}
sslm_status sslm_tokenize(sslm_model, const char*, int32_t*, int32_t*) { return SSLM_INVALID_ARGUMENT; }
sslm_status sslm_schema_lookup(sslm_model, const char*, sslm_schema* out) {
	if (out) *out = nullptr;
	return SSLM_SCHEMA_NOT_FOUND;
}
size_t sslm_schema_count(sslm_model) { return 0; }
sslm_status sslm_schema_name(sslm_model, int32_t, char*, size_t*) { return SSLM_INVALID_ARGUMENT; }
sslm_status sslm_seq_set_schema(sslm_seq, sslm_schema) { return SSLM_INVALID_ARGUMENT; }
sslm_status sslm_prefix_set_schema(sslm_prefix, sslm_schema) { return SSLM_INVALID_ARGUMENT; }
sslm_status sslm_detokenize_stream(sslm_model, sslm_detok_state*, const int32_t*, int32_t, char*, int32_t* out_n) {
	if (out_n) *out_n = 0;
	return SSLM_INVALID_ARGUMENT;
}

// ---- standalone GEMM entry points (BASELINE configuration 0 and verification) ----
namespace {
struct StandaloneCtx {
	hipStream_t stream = nullptr;
	std::vector<void*> owned;
	int32_t* f = nullptr;
	size_t f_n = 0;
	uint32_t* mx = nullptr;
	size_t mx_n = 0;
	TokenInfo* tok = nullptr;
	Scale* in = nullptr;
	int cap_m = 0;
	std::mutex mu;
};
StandaloneCtx g_sa;

void sa_reserve(int m, int n) {
	if (!g_sa.stream) ck(hipStreamCreate(&g_sa.stream));

	const size_t mn = (size_t)m * n;
	if (mn > g_sa.f_n) {
		g_sa.f = dalloc<int32_t>(mn, &g_sa.owned);
		g_sa.f_n = mn;
	}
	if ((size_t)n > g_sa.mx_n) {
		g_sa.mx = dalloc<uint32_t>((size_t)(n + 15) / 16 * kPartLd, &g_sa.owned);
		g_sa.mx_n = n;
	}
	if (m > g_sa.cap_m) {
		g_sa.tok = dalloc<TokenInfo>(m, &g_sa.owned);
		g_sa.in = dalloc<Scale>(m, &g_sa.owned);
		std::vector<TokenInfo> ti(m);
		for (int t = 0; t < m; ++t) ti[t] = TokenInfo{0, t, 0};
		ck(hipMemcpy(g_sa.tok, ti.data(), m * sizeof(TokenInfo), hipMemcpyHostToDevice));
		g_sa.cap_m = m;
	}
}

GemmArgs sa_args(const int8_t* a, const int8_t* w, int m, int n, int k) {
	GemmArgs g{};
	g.a = a;
	g.w = w;
	g.M = m;
	g.N = n;
	g.K = k;
	g.lda = k;
	g.epi.tok = g_sa.tok;
	return g;
}
}  // namespace

sslm_status sslm_hip_gemm_requant(const int8_t* a, const int8_t* w, const int32_t* fold, int32_t m, int32_t n,
                                  int32_t k, int64_t in_m, int64_t in_e, int64_t site_m, int64_t site_e,
                                  int8_t* out_codes, int64_t* out_me, int32_t* out_status) {
	if (!a || !w || !fold || !out_codes || !out_me || !out_status || m < 1 || m > kPartLd || n < 1 || k < 16 ||
	    k % 16 || n % 16)
		return SSLM_INVALID_ARGUMENT;
	return guarded([&]() -> sslm_status {
		std::lock_guard<std::mutex> lk(g_sa.mu);
		sa_reserve(m, n);
		std::vector<Scale> in(m, Scale{in_m, in_e});
		ck(hipMemcpyAsync(g_sa.in, in.data(), m * sizeof(Scale), hipMemcpyHostToDevice, g_sa.stream));
		ck(hipMemsetAsync(out_status, 0, (size_t)m * 4, g_sa.stream));
		GemmArgs g = sa_args(a, w, m, n, k);
		g.epi.status = out_status;
		g.epi.nseg = 1;
		g.epi.seg[0] = funnel_seg(0, n, g_sa.f, n, g_sa.mx, fold, nullptr);
		{
			ProfScope p(g_sa.stream, kProfGemm, (int64_t)n * k + (int64_t)m * k + 12LL * n + 4LL * m * n,
			            2LL * m * n * k);
			sslm_launch::gemm(g, g_sa.stream);
			ck(hipGetLastError());
		}
		sslm_launch::FunnelArgs fa{};
		fa.M = m;
		fa.N = n;
		fa.tok = g_sa.tok;
		fa.f = g_sa.f;
		fa.ld_f = n;
		fa.maxpart = g_sa.mx;
		fa.ntiles = (n + 15) / 16;
		fa.incoming = g_sa.in;
		fa.site = Scale{site_m, site_e};
		fa.out = out_codes;
		fa.out_scale = (Scale*)out_me;
		fa.layer = 0;
		fa.status = out_status;
		{
			ProfScope p(g_sa.stream, kProfRow, 4LL * m * n + (int64_t)m * n, 0);
			sslm_launch::funnel(fa, g_sa.stream);
			ck(hipGetLastError());
		}
		ck(hipStreamSynchronize(g_sa.stream));
		prof_collect();
		return SSLM_OK;
	});
}

sslm_status sslm_hip_gemm_i32(const int8_t* a, const int8_t* w, int32_t m, int32_t n, int32_t k, int32_t* out) {
	if (!a || !w || !out || m < 1 || m > kPartLd || n < 1 || k < 16 || k % 16) return SSLM_INVALID_ARGUMENT;
	return guarded([&]() -> sslm_status {
		std::lock_guard<std::mutex> lk(g_sa.mu);
		sa_reserve(m, n);
		GemmArgs g = sa_args(a, w, m, n, k);
		g.epi.raw_out = out;
		{
			ProfScope p(g_sa.stream, kProfGemm, (int64_t)n * k + (int64_t)m * k + 4LL * m * n, 2LL * m * n * k);
			sslm_launch::gemm(g, g_sa.stream);
			ck(hipGetLastError());
		}
		ck(hipStreamSynchronize(g_sa.stream));
		prof_collect();
		return SSLM_OK;
	});
}

void* sslm_hip_device_alloc(size_t bytes) {
	void* p = nullptr;
	if (hipMalloc(&p, bytes ? bytes : 1) != hipSuccess) return nullptr;
	return p;
}

void sslm_hip_device_free(void* p) {
	if (p) (void)hipFree(p);
}

sslm_status sslm_hip_copy(void* dst, const void* src, size_t bytes, int kind) {
	if (!dst || !src) return SSLM_INVALID_ARGUMENT;
	const hipMemcpyKind k = kind == 0 ? hipMemcpyHostToDevice : (kind == 1 ? hipMemcpyDeviceToHost : hipMemcpyDeviceToDevice);
	return hipMemcpy(dst, src, bytes, k) == hipSuccess ? SSLM_OK : SSLM_INVALID_ARGUMENT;
}

sslm_status sslm_hip_synchronize(void) { return hipDeviceSynchronize() == hipSuccess ? SSLM_OK : SSLM_INVALID_ARGUMENT; }

// ---- profiling ----
void sslm_hip_profile_enable(int on) { g_prof.on = on != 0; }
void sslm_hip_profile_reset(void) {
	for (int i = 0; i < SSLM_HIP_PROFILE_CLASSES; ++i) {
		g_prof.ms[i] = 0;
		g_prof.launches[i] = g_prof.bytes[i] = g_prof.ops[i] = 0;
	}
}
void sslm_hip_profile_read(double* ms, int64_t* launches, int64_t* bytes, int64_t* ops, int classes) {
	prof_collect();
	for (int i = 0; i < classes && i < SSLM_HIP_PROFILE_CLASSES; ++i) {
		if (ms) ms[i] = g_prof.ms[i];
		if (launches) launches[i] = g_prof.launches[i];
		if (bytes) bytes[i] = g_prof.bytes[i];
		if (ops) ops[i] = g_prof.ops[i];
	}
}

}  // extern "C"
