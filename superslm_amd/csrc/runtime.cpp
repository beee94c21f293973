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
#include <deque>
#include <functional>
#include <memory>
#include <map>
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
constexpr int kTracks = 4;           // concurrent token groups of one decode step
constexpr int kTrackTokens = 128;    // tokens per launch on tracks 1..kTracks-1
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
		int64_t key;  // launch shape, 0 for none
	};
	struct ShapeAgg {
		double ms = 0;
		int64_t launches = 0, bytes = 0, ops = 0;
	};
	std::vector<Pending> pending;
	std::map<int64_t, ShapeAgg> shapes;
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
	int64_t key;
	ProfScope(hipStream_t s_, int c, int64_t bytes, int64_t ops, int64_t shape_key = 0) : s(s_), cls(c), key(shape_key) {
		if (!g_prof.on) return;
		a = prof_event();
		ck(hipEventRecord(a, s));
		g_prof.bytes[c] += bytes;
		g_prof.ops[c] += ops;
		g_prof.launches[c] += 1;
		if (key) {
			auto& sa = g_prof.shapes[key];
			sa.launches += 1;
			sa.bytes += bytes;
			sa.ops += ops;
		}
	}
	~ProfScope() {
		if (!a) return;
		hipEvent_t b = prof_event();
		(void)hipEventRecord(b, s);
		g_prof.pending.push_back({a, b, cls, key});
	}
};

bool prof_enabled() { return g_prof.on; }

// (class, M, N, K) packed as class << 56 | M << 40 | N << 20 | K (M < 65536, N and K < 2^20)
int64_t profile_shape_key(int cls, int64_t M, int64_t N, int64_t K) {
	return ((int64_t)cls << 56) | (M << 40) | (N << 20) | K;
}

void prof_collect() {
	if (g_prof.pending.empty()) return;
	for (auto& p : g_prof.pending) {
		(void)hipEventSynchronize(p.b);
		float ms = 0;
		(void)hipEventElapsedTime(&ms, p.a, p.b);
		g_prof.ms[p.cls] += ms;
		if (p.key) g_prof.shapes[p.key].ms += ms;
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
	int8_t *p_qkv, *p_o, *p_gu, *p_down;  // packed decode copies (sslm_launch::pack_gemv), or null
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

// Scratch of one launch sequence: a stream and every per-token buffer the layer loop and the
// head use.  Several tracks run independent token groups of one decode step concurrently.
struct Track {
	hipStream_t stream = nullptr;
	int capacity = 0;  // tokens per launch
	int32_t attn_wcap = 0;  // decode: the grouped attention's score-row length for the current unit
	TokenInfo* tok;
	int32_t *tok_ids, *ident, *slot_idx, *out_tokens;
	int8_t *hid_chunk, *normed, *q_rot, *ctx, *attn_stream, *mlp_normed, *act, *final_codes;
	Scale *hid_chunk_scale, *normed_scale, *q_scale, *ctx_scale, *attn_stream_scale, *mlp_scale, *act_scale,
	    *final_scale;
	int64_t *normed_recip, *mlp_recip, *kv_f, *attn_scratch;
	int32_t *q_f, *ctx_f, *o_f, *gu_f, *down_f;
	uint32_t *mx_q, *mx_ctx, *mx_o, *mx_gu, *mx_down;  // per (16-column tile, token) partial maxima
	unsigned long long* argmax_key;                    // [token][tile], head tracks only
	int32_t* raw_part;  // split-K partial planes, consumed by the next row kernel
	int32_t* act_prod;       // decode tracks: SiLU products of the sliced mlp_act [64, I]
	uint32_t* act_maxpart;   // its per-slice maxima
	Scale* gu_scale;         // its gate / up scales [64, 2]
	int8_t* kv_stage;    // prefill tracks: landed K/V rows awaiting kv_commit [T][2 * KVH]
	uint32_t* sat_stage;  // prefill tracks: their clamp counts [T]
	int8_t* lora_u[3];
	TokenInfo* lg_tok;    // head tracks: tokens of the joined final norm + head
	int32_t* lg_slot;
	const uint8_t** lg_mask;  // head tracks: per token its schema mask page in HBM, or null
	hipEvent_t done = nullptr;
	hipEvent_t fork = nullptr;
	bool prefill = false;    // carries prefill spans (one sequence, consecutive positions)
	std::vector<void*> own;  // device buffers of this track
	int gen = 0;             // bumped when the buffers are reallocated (graph keys carry it)
};

// Damped-greedy anti-LM (src/damped_greedy_antilm.cpp): for each order n in 1..max_order, the
// counts of tokens that followed each (n-1)-token context of the generated history, and the
// history itself.  Only lookups by context are made, so an ordered map serves (no iteration
// order reaches any result).
struct AntiLm {
	struct Entry {
		std::map<int32_t, int64_t> counts;
		int64_t total = 0;
	};
	int order = 0;
	std::vector<std::map<std::vector<int32_t>, Entry>> tables;
	std::vector<int32_t> history;

	void reset(int max_order) {
		order = max_order;
		tables.assign(max_order > 0 ? max_order : 0, {});
		history.clear();
	}
	const Entry* context(int n) const {  // the table entry of order n's current context
		const size_t len = (size_t)n - 1;
		if (len > history.size()) return nullptr;
		const std::vector<int32_t> ctx(history.end() - (long)len, history.end());
		auto it = tables[n - 1].find(ctx);
		return it == tables[n - 1].end() ? nullptr : &it->second;
	}
	// AntiLmUpdate, :129-152
	void update(int32_t token) {
		for (int n = 1; n <= order; ++n) {
			const size_t len = (size_t)n - 1;
			if (len > history.size()) continue;
			Entry& e = tables[n - 1][std::vector<int32_t>(history.end() - (long)len, history.end())];
			e.counts[token] += 1;
			e.total += 1;
		}
		history.push_back(token);
	}
	// AntiLmPenalize, :160-228: p_omega in Q15 per candidate, a beta^(max_order - n) weighted
	// mix over the orders whose context was seen (weights normalized, the last takes the rest)
	void penalize(const int32_t* cand, size_t k, int64_t* out) const {
		constexpr int64_t kBetaQ15 = 29491;  // round(0.9 * 2^15)
		auto pow_q15 = [](int64_t b, int ex) {
			int64_t r = (int64_t)1 << 15;
			for (int i = 0; i < ex; ++i) r = (r * b) >> 15;
			return r;
		};
		for (size_t c = 0; c < k; ++c) out[c] = 0;
		int active = 0;
		int64_t raw_sum = 0;
		for (int n = 1; n <= order; ++n)
			if (context(n)) {
				++active;
				raw_sum += pow_q15(kBetaQ15, order - n);
			}
		if (active == 0) return;
		int idx = 0;
		int64_t norm_sum = 0;
		for (int n = 1; n <= order; ++n) {
			const Entry* e = context(n);
			if (!e) continue;
			++idx;
			const int64_t w = idx == active ? ((int64_t)1 << 15) - norm_sum
			                                : (pow_q15(kBetaQ15, order - n) << 15) / raw_sum;
			norm_sum += w;
			for (size_t c = 0; c < k; ++c) {
				auto f = e->counts.find(cand[c]);
				const int64_t count = f == e->counts.end() ? 0 : f->second;
				out[c] += (w * ((count << 15) / e->total)) >> 15;
			}
		}
		for (size_t c = 0; c < k; ++c) out[c] = std::min<int64_t>(std::max<int64_t>(out[c], 0), (int64_t)1 << 15);
	}
};

// SCM1 schema masks (include/superslm/schema_masks.h): per schema a DFA over token ids -- one
// vocabulary bitmask page per state (bit t set iff the state has a transition on token t), the
// CSR transition rows (token ascending) and the sorted accepting set.  The tables point into the
// artifact bytes, which outlive the model.
struct SchemaEntry {
	std::string name;
	uint64_t name_hash = 0;  // FNV-1a 64 of the name
	uint32_t states = 0, accepting_count = 0, transitions = 0;
	const uint8_t* pages = nullptr;    // states x page_bytes
	const uint8_t* offsets = nullptr;  // states + 1 LE u32
	const uint8_t* accepting = nullptr;
	const uint8_t* trans = nullptr;    // (token, next) LE u32 pairs
};

struct sslm_schema_s {
	sslm_model model = nullptr;
	uint32_t index = 0;
};

struct sslm_model_s {
	Artifact art;
	ModelConfig c;
	int H, L, NH, NKV, D, I, V, KVH;
	int64_t cap;
	size_t block_bytes;
	std::vector<void*> owned;
	std::vector<DevLayer> layers;
	int8_t *embed, *head;
	int8_t* head_pk = nullptr;  // packed decode copy of the LM head, or null
	// sslm_hip_debug_capture: every site of every layer of the last launch sequence of at most
	// dbg_tokens tokens, codes [layer][site][token][dbg_ld] and scales [layer][site][token]
	int dbg_tokens = 0, dbg_ld = 0;
	int8_t* dbg_codes = nullptr;
	Scale* dbg_scales = nullptr;
	int32_t *final_gain, *silu;
	int64_t *rope_cos, *rope_sin;
	Scale embed_site, final_site;
	int64_t ln2_q, b_q, ca_q;
	// damped greedy: i-exp triple of the artifact's logit scale (src/sslm_abi.cpp:1172-1185)
	bool dg_available = false;
	int64_t dg_q_ln2 = 0, dg_q_b = 0, dg_q_c = 0;
	int32_t* logits = nullptr;  // [kMaxTokens, V] raw head rows, allocated on first use
	int2* topk = nullptr;       // [kMaxTokens, kTopKMax] damped greedy's device candidates
	std::vector<SchemaEntry> schemas;
	std::vector<sslm_schema_s> schema_handles;
	uint32_t page_bytes = 0;  // (V + 7) / 8
	uint8_t* d_pages = nullptr;     // every schema's mask pages, in HBM
	std::vector<size_t> page_off;   // per schema: offset of its pages in d_pages
	// per-slot sequence state
	int8_t* stream_codes;   // [kSlotCapacity, H]
	Scale* stream_scale;    // [kSlotCapacity]
	unsigned long long* sat;  // [kSlotCapacity]
	int32_t* status;        // [kSlotCapacity]
	int32_t* head_status;   // [kSlotCapacity] attention-stage refusals awaiting the ctx funnel
	int8_t* snap_codes;     // [kSlotCapacity, H] stream rows as a decode call found them
	Scale* snap_scale;      // [kSlotCapacity]
	unsigned long long* snap_sat;  // [kSlotCapacity]
	int8_t* snap_kv;        // [kSlotCapacity, L * 2 * KVH] K/V rows at the call's position
	std::vector<int> free_slots;
	std::vector<Track> tracks;  // tracks[0]: the LM head; all: decode token groups
	Track prefill;              // prefill spans: capacity grown on demand up to kMaxPrefillTokens
	std::map<std::string, hipGraphExec_t> graphs;  // captured submissions by shape
	std::map<std::string, int> graph_seen;         // prefill shapes seen (captured on a repeat)
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
	int64_t forced_token_count = 0;
	AntiLm anti_lm;  // damped-greedy n-gram state (order 0: none)
	sslm_schema schema = nullptr;       // bound schema
	uint32_t walk = 0xFFFFFFFFu;        // DFA walk state (0xFFFFFFFF: no schema bound)
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

// sequence blob constants (src/sslm_abi.cpp:102, :2585-2618)
constexpr uint8_t kBlobMagic[4] = {'S', 'S', 'B', '3'};
constexpr uint8_t kBlobMagicV2[4] = {'S', 'S', 'B', '2'};
constexpr size_t kBlobHeader = 120, kBlobHeaderV2 = 108;
constexpr uint32_t kWalkUnused = 0xFFFFFFFFu;  // DFA walk state of a sequence with no schema bound

void put32(uint8_t* p, uint32_t v) {
	for (int i = 0; i < 4; ++i) p[i] = (uint8_t)(v >> (8 * i));
}
void put64(uint8_t* p, uint64_t v) {
	for (int i = 0; i < 8; ++i) p[i] = (uint8_t)(v >> (8 * i));
}
uint32_t get32(const uint8_t* p) {
	uint32_t v = 0;
	for (int i = 0; i < 4; ++i) v |= (uint32_t)p[i] << (8 * i);
	return v;
}
uint64_t get64(const uint8_t* p) {
	uint64_t v = 0;
	for (int i = 0; i < 8; ++i) v |= (uint64_t)p[i] << (8 * i);
	return v;
}

uint64_t fnv1a64(const char* p, size_t n) {
	uint64_t h = 14695981039346656037ull;
	for (size_t i = 0; i < n; ++i) {
		h ^= (uint8_t)p[i];
		h *= 1099511628211ull;
	}
	return h;
}

// SchemaMasksTable::Parse (include/superslm/schema_masks.h): 24-byte header ("SCM1", version 1,
// schema count in [1, 65536], vocab = the config's, name blob length, reserved 0), 56-byte
// descriptors, the name blob, then per schema four non-overlapping blocks after the manifest
// (mask pages, state offsets, accepting set, transitions) with: offsets[0] = 0, nondecreasing,
// offsets[states] = transitions; accepting strictly ascending below `states`; each CSR row's
// tokens strictly ascending, tokens < vocab, next states < states; and every mask bit equal to
// the existence of the transition.  Returns false on any violation.
bool parse_schemas(const uint8_t* d, uint64_t size, uint32_t vocab, std::vector<SchemaEntry>* out) {
	out->clear();
	if (size < 24 || memcmp(d, "SCM1", 4) != 0 || get32(d + 4) != 1) return false;
	const uint32_t count = get32(d + 8), v = get32(d + 12), blob = get32(d + 16);
	if (get32(d + 20) != 0 || count == 0 || count > 65536 || v == 0 || v != vocab) return false;
	const uint64_t manifest_end = 24 + (uint64_t)count * 56 + blob;
	if (manifest_end > size) return false;
	const uint64_t blob_off = manifest_end - blob, page = ((uint64_t)v + 7) / 8;
	struct Span {
		uint64_t off, len;
	};
	std::vector<Span> used;
	auto overlaps = [](const Span& a, const Span& b) { return a.off < b.off + b.len && b.off < a.off + a.len; };
	for (uint32_t i = 0; i < count; ++i) {
		const uint8_t* e = d + 24 + (uint64_t)i * 56;
		const uint32_t name_off = get32(e), name_len = get32(e + 4), states = get32(e + 8), acc = get32(e + 12),
		               trans = get32(e + 16);
		if (get32(e + 20) != 0) return false;
		if (name_len == 0 || (uint64_t)name_off + name_len > blob) return false;
		SchemaEntry se;
		se.name.assign((const char*)d + blob_off + name_off, name_len);
		for (auto& o : *out)
			if (o.name == se.name) return false;
		if (states == 0 || states > 1048576 || acc > states || trans > 16777216) return false;
		const Span blocks[4] = {{get64(e + 24), (uint64_t)states * page},
		                        {get64(e + 32), ((uint64_t)states + 1) * 4},
		                        {get64(e + 40), (uint64_t)acc * 4},
		                        {get64(e + 48), (uint64_t)trans * 8}};
		for (const Span& b : blocks)
			if (b.off > UINT64_MAX - b.len || b.off < manifest_end || b.off + b.len > size) return false;
		for (const Span& b : blocks)
			for (const Span& u : used)
				if (overlaps(b, u)) return false;
		for (int a = 0; a < 4; ++a)
			for (int b = a + 1; b < 4; ++b)
				if (overlaps(blocks[a], blocks[b])) return false;
		for (const Span& b : blocks) used.push_back(b);
		const uint8_t* offs = d + blocks[1].off;
		if (get32(offs) != 0 || get32(offs + (size_t)states * 4) != trans) return false;
		for (uint32_t st = 0; st < states; ++st)
			if (get32(offs + (size_t)st * 4) > get32(offs + (size_t)(st + 1) * 4)) return false;
		const uint8_t* accp = d + blocks[2].off;
		for (uint32_t a = 0; a < acc; ++a) {
			const uint32_t x = get32(accp + (size_t)a * 4);
			if (x >= states || (a > 0 && x <= get32(accp + (size_t)(a - 1) * 4))) return false;
		}
		const uint8_t* tr = d + blocks[3].off;
		const uint8_t* pages = d + blocks[0].off;
		for (uint32_t st = 0; st < states; ++st) {
			const uint32_t r0 = get32(offs + (size_t)st * 4), r1 = get32(offs + (size_t)(st + 1) * 4);
			for (uint32_t k = r0; k < r1; ++k) {
				const uint32_t tok = get32(tr + (size_t)k * 8), nx = get32(tr + (size_t)k * 8 + 4);
				if (tok >= v || nx >= states || (k > r0 && tok <= get32(tr + (size_t)(k - 1) * 8))) return false;
			}
			const uint8_t* pg = pages + (size_t)st * page;
			uint32_t cur = r0;
			for (uint32_t t = 0; t < v; ++t) {
				const bool bit = (pg[t >> 3] >> (t & 7)) & 1u;
				bool in_row = false;
				if (cur < r1 && get32(tr + (size_t)cur * 8) == t) {
					in_row = true;
					++cur;
				}
				if (bit != in_row) return false;
			}
		}
		se.name_hash = fnv1a64(se.name.data(), se.name.size());
		se.states = states;
		se.accepting_count = acc;
		se.transitions = trans;
		se.pages = pages;
		se.offsets = offs;
		se.accepting = accp;
		se.trans = tr;
		out->push_back(std::move(se));
	}
	return true;
}

// SchemaMasksTable::Transition: binary search of state's CSR row
bool schema_next(const SchemaEntry& e, uint32_t state, uint32_t token, uint32_t* next) {
	uint32_t lo = get32(e.offsets + (size_t)state * 4), hi = get32(e.offsets + (size_t)(state + 1) * 4);
	while (lo < hi) {
		const uint32_t mid = lo + (hi - lo) / 2;
		const uint32_t t = get32(e.trans + (size_t)mid * 8);
		if (t == token) {
			*next = get32(e.trans + (size_t)mid * 8 + 4);
			return true;
		}
		if (t < token) lo = mid + 1;
		else hi = mid;
	}
	return false;
}

bool schema_accepting(const SchemaEntry& e, uint32_t state) {  // src/sslm_abi.cpp:2488-2503
	uint32_t lo = 0, hi = e.accepting_count;
	while (lo < hi) {
		const uint32_t mid = lo + (hi - lo) / 2;
		const uint32_t v = get32(e.accepting + (size_t)mid * 4);
		if (v == state) return true;
		if (v < state) lo = mid + 1;
		else hi = mid;
	}
	return false;
}

// ------------------------------------------------------------------------------------------
// launch helpers
// ------------------------------------------------------------------------------------------
GemmArgs gemm_args(sslm_model m, Track& w, const int8_t* a, int M, int lda, const int8_t* wt, int N, int K,
                   const int8_t* wpk = nullptr) {
	GemmArgs g{};
	g.a = a;
	g.w = wt;
	g.wp = wpk;
	g.M = M;
	g.N = N;
	g.K = K;
	g.lda = lda;
	g.epi.tok = w.tok;
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

void run_gemm(sslm_model m, Track& w, const GemmArgs& g, int cls) {
	const int64_t out_bytes = g.epi.argmax_key ? 0 : (int64_t)g.M * g.N * 4;
	ProfScope p(w.stream, cls, (int64_t)g.N * g.K + (int64_t)g.M * g.K + 12LL * g.N + out_bytes,
	            2LL * g.M * g.N * g.K, profile_shape_key(cls, g.M, g.N, g.K));
	sslm_launch::gemm(g, w.stream);
	ck(hipGetLastError());
}

// Decode projections (and prefill GEMMs that split K) hand their raw partial planes to the next
// row kernel, which applies the epilogue; call once g.epi is complete.  Returns a null RawIn
// otherwise.  `allow_multi` / `allow_single`: the consumer's raw variant for several planes /
// one plane holds its row in registers without (much) spilling.
RawIn split_raw(sslm_model m, Track& w, GemmArgs& g, bool allow_multi, bool allow_single) {
	RawIn r{};
	if (!w.raw_part) return r;
	bool lora = false;
	for (int i = 0; i < g.epi.nseg; ++i) lora = lora || g.epi.seg[i].lora_b;
	int splits = 1;
	// A decode GEMV always hands its raw accumulators to the consumer, which applies the
	// epilogue on the row: in the GEMV the epilogue's stores and waits sit behind the weight
	// stream.  A prefill GEMM keeps its own epilogue unless it splits K.  The flags say which
	// raw consumers fit their register budget (several planes / one plane).
	if (sslm_launch::gemv_eligible(g.M, g.K)) {
		splits = allow_multi ? sslm_launch::gemv_raw_splits(g) : 1;
		if (splits == 1 && !allow_single) return r;
	} else {
		if (!allow_multi || lora || !sslm_launch::prefill_mfma_k(g.K)) return r;
		const PrefillPlan pp = sslm_launch::prefill_plan(g.M, g.N, g.K, true);
		splits = pp.splits;
		if (pp.narrow && !allow_single) return r;  // the 64 x 64-tile kernel writes raw only
		if (splits <= 1 && !pp.narrow) return r;
	}
	r.part = w.raw_part;
	r.splits = splits;
	r.ld = g.N;
	r.epi = g.epi;
	if (splits > 1) {
		g.splits = splits;
		g.split_part = w.raw_part;
	} else {
		g.epi.raw_out = w.raw_part;  // plane 0 of [splits][M][N]
	}
	return r;
}

void attach_lora(sslm_model m, Track& w, sslm_adapter ad, int layer, int proj, Segment* seg, int slot_u) {
	if (!ad) return;
	const AdapterProj& p = ad->proj[(size_t)layer * 7 + proj];
	if (!p.a) return;
	seg->lora_b = p.b;
	seg->lora_dfold = p.dfold;
	seg->lora_u = w.lora_u[slot_u];
}

void run_lora_u(sslm_model m, Track& w, sslm_adapter ad, int layer, const int* projs, int n, const int8_t* x, int M, int K) {
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
		a.u[cnt] = w.lora_u[i];
		++cnt;
	}
	if (!cnt) return;
	a.nproj = cnt;
	ProfScope ps(w.stream, kProfLora, (int64_t)cnt * ad->rank * K + (int64_t)M * K, 2LL * M * cnt * ad->rank * K);
	sslm_launch::lora_u(a, w.stream);
	ck(hipGetLastError());
}

// The projections' GEMM arguments (forward_sites.cpp:1699-1735, :1907-1914, :1938-1955,
// :1969-1977), shared by the layer loop and the GEMV benchmark entry.  split_raw() decides
// whether the consumer adds split-K planes.
struct ProjArgs {
	GemmArgs g;
	RawIn raw;
};

ProjArgs qkv_args(sslm_model m, Track& w, int l, int M, sslm_adapter ad, bool fused) {
	const DevLayer& lw = m->layers[l];
	const int H = m->H, KVH = m->KVH;
	GemmArgs g = gemm_args(m, w, w.normed, M, H, lw.w_qkv, H + 2 * KVH, H, lw.p_qkv);
	g.epi.layer = l;
	g.epi.in_recip = w.normed_recip;
	g.epi.in_scale = w.normed_scale;
	g.epi.rank = ad ? (int)ad->rank : 0;
	g.epi.nseg = 3;
	g.epi.seg[0] = funnel_seg(0, H, w.q_f, H, w.mx_q, lw.f_qkv, lw.b_q);
	Segment sk{};
	sk.n_begin = H;
	sk.n_end = H + KVH;
	sk.mode = kSegWide;
	sk.out = w.kv_f;
	sk.ld_out = 2 * KVH;
	sk.fold = lw.f_qkv + 3 * H;
	sk.bias = lw.b_k;
	Segment sv = sk;
	sv.n_begin = H + KVH;
	sv.n_end = H + 2 * KVH;
	sv.out = w.kv_f + KVH;
	sv.fold = lw.f_qkv + 3 * (H + KVH);
	sv.bias = lw.b_v;
	g.epi.seg[1] = sk;
	g.epi.seg[2] = sv;
	attach_lora(m, w, ad, l, 0, &g.epi.seg[0], 0);
	attach_lora(m, w, ad, l, 1, &g.epi.seg[1], 1);
	attach_lora(m, w, ad, l, 2, &g.epi.seg[2], 2);
	ProjArgs pa{g, RawIn{}};
	// the fused decode attention reads the funnel epilogue's outputs (q tile maxima, K/V wide)
	if (!fused) pa.raw = split_raw(m, w, pa.g, H <= 4096, true);
	return pa;
}

ProjArgs o_args(sslm_model m, Track& w, int l, int M, sslm_adapter ad) {
	const DevLayer& lw = m->layers[l];
	const int H = m->H;
	GemmArgs g = gemm_args(m, w, w.ctx, M, H, lw.w_o, H, H, lw.p_o);
	g.epi.layer = l;
	g.epi.rank = ad ? (int)ad->rank : 0;
	g.epi.nseg = 1;
	g.epi.seg[0] = funnel_seg(0, H, w.o_f, H, w.mx_o, lw.f_o, nullptr);
	attach_lora(m, w, ad, l, 3, &g.epi.seg[0], 0);
	ProjArgs pa{g, RawIn{}};
	pa.raw = split_raw(m, w, pa.g, H <= 6144, true);
	return pa;
}

ProjArgs gu_args(sslm_model m, Track& w, int l, int M, sslm_adapter ad) {
	const DevLayer& lw = m->layers[l];
	const int H = m->H, I = m->I;
	GemmArgs g = gemm_args(m, w, w.mlp_normed, M, H, lw.w_gu, 2 * I, H, lw.p_gu);
	g.epi.layer = l;
	g.epi.rank = ad ? (int)ad->rank : 0;
	g.epi.nseg = 2;
	g.epi.seg[0] = funnel_seg(0, I, w.gu_f, 2 * I, w.mx_gu, lw.f_gu, nullptr);
	g.epi.seg[1] = funnel_seg(I, 2 * I, w.gu_f + I, 2 * I, w.mx_gu, lw.f_gu + 3 * I, nullptr);
	attach_lora(m, w, ad, l, 4, &g.epi.seg[0], 0);
	attach_lora(m, w, ad, l, 5, &g.epi.seg[1], 1);
	ProjArgs pa{g, RawIn{}};
	pa.raw = split_raw(m, w, pa.g, I <= 4096, false);
	return pa;
}

ProjArgs down_args(sslm_model m, Track& w, int l, int M, sslm_adapter ad) {
	const DevLayer& lw = m->layers[l];
	const int H = m->H, I = m->I;
	GemmArgs g = gemm_args(m, w, w.act, M, I, lw.w_down, H, I, lw.p_down);
	g.epi.layer = l;
	g.epi.rank = ad ? (int)ad->rank : 0;
	g.epi.nseg = 1;
	g.epi.seg[0] = funnel_seg(0, H, w.down_f, H, w.mx_down, lw.f_down, nullptr);
	attach_lora(m, w, ad, l, 6, &g.epi.seg[0], 0);
	ProjArgs pa{g, RawIn{}};
	pa.raw = split_raw(m, w, pa.g, H <= 6144, true);
	return pa;
}

GemmArgs head_args(sslm_model m, Track& w, int M, const TokenInfo* tok) {
	GemmArgs g = gemm_args(m, w, w.final_codes, M, m->H, m->head, m->V, m->H, m->head_pk);
	g.epi.tok = tok;
	g.epi.argmax_key = w.argmax_key;
	g.epi.key_ld = (m->V + 15) / 16;
	g.epi.layer = m->L;
	return g;
}

// Attention arguments shared by the fused (decode) and the two-kernel (prefill) paths.
sslm_launch::AttnArgs attn_args(sslm_model m, Track& w, int l, int M) {
	const DevLayer& lw = m->layers[l];
	sslm_launch::AttnArgs a{};
	a.M = M;
	a.H = m->H;
	a.NH = m->NH;
	a.NKV = m->NKV;
	a.D = m->D;
	a.cap = m->cap;
	a.wcap = w.attn_wcap > 0 ? w.attn_wcap : sslm_launch::group_width_cap(m->cap, m->cap);
	a.row_halves = sslm_launch::group_row_halves(M, m->NKV, m->NH / m->NKV);
	a.tok = w.tok;
	a.khead_m = lw.khead_m;
	a.khead_e = lw.khead_e;
	a.ctx_fold = lw.ctx_fold;
	a.kv_pool = m->pool_dev;
	a.block_bytes = (int64_t)m->block_bytes;
	a.layer = l;
	a.ln2_q = m->ln2_q;
	a.b_q = m->b_q;
	a.ca_q = m->ca_q;
	a.ctx_f = w.ctx_f;
	a.ctx_maxpart = w.mx_ctx;
	a.scratch = w.attn_scratch;
	a.status = m->status;
	a.head_status = m->head_status;
	return a;
}

bool fused_attention_enabled() {
	static const bool on = [] {
		const char* e = getenv("SSLM_HIP_FUSED_ATTN");
		return !(e && e[0] == '0');
	}();
	return on;
}

// Sites of the debug capture, in the oracle's trace numbering (site 6 holds q after RoPE).
constexpr int kDbgSites = 11;
enum DbgSite {
	kDbgAttnNorm = 0, kDbgCtx = 1, kDbgAttnRes = 2, kDbgMlpNorm = 3, kDbgAct = 4, kDbgMlpRes = 5, kDbgQRot = 6,
	kDbgO = 7, kDbgGate = 8, kDbgUp = 9, kDbgDown = 10
};

bool dbg_on(sslm_model m, int M) { return m->dbg_codes && M <= m->dbg_tokens; }

sslm_launch::SiteTap dbg_tap(sslm_model m, int l, int site) {
	const size_t cell = (size_t)l * kDbgSites + site;
	return sslm_launch::SiteTap{m->dbg_codes + cell * m->dbg_tokens * m->dbg_ld, m->dbg_scales + cell * m->dbg_tokens,
	                            m->dbg_ld};
}

void dbg_gather(sslm_model m, Track& w, int l, int site, const int8_t* src, const Scale* sc, const int32_t* idx, int n,
                int M) {
	const sslm_launch::SiteTap tp = dbg_tap(m, l, site);
	sslm_launch::debug_gather(src, sc, idx, n, M, tp.codes, tp.scale, tp.ld, w.stream);
	ck(hipGetLastError());
}

// The stream (committed hidden state) a launch sequence reads and commits: decode batches use
// the per-slot state, prefill chunks the chunk rows.
struct StreamRef {
	int8_t* codes;
	Scale* scale;
	const int32_t* idx;
};

// Layers [l0, l1) for M tokens whose TokenInfo is already on the device.
// `decode`: every token belongs to a different sequence (a decode step), so attention may take
// the fused path.
void run_layers(sslm_model m, Track& w, int M, StreamRef st, int l0, int l1, sslm_adapter ad, bool decode) {
	const int H = m->H, I = m->I, KVH = m->KVH;
	hipStream_t s = w.stream;
	{
		ProfScope p(s, kProfRow, 0, 0);
		sslm_launch::RowNormArgs a{st.codes, st.idx, H, m->layers[l0].attn_gain, m->layers[l0].attn_norm,
		                           w.normed, w.normed_scale, w.normed_recip};
		sslm_launch::rmsnorm(a, M, H, w.tok, m->status, l0, s);
		ck(hipGetLastError());
	}
	const bool fused = decode && sslm_launch::gemv_eligible(M, H) && fused_attention_enabled();
	const bool dbg = dbg_on(m, M);
	for (int l = l0; l < l1; ++l) {
		const DevLayer& lw = m->layers[l];
		RawIn raw{};  // the last projection's split-K partials, when it split
		if (dbg) dbg_gather(m, w, l, kDbgAttnNorm, w.normed, w.normed_scale, nullptr, H, M);
		// q | k | v projection (forward_sites.cpp:1699-1735)
		{
			const int pj[3] = {0, 1, 2};
			run_lora_u(m, w, ad, l, pj, 3, w.normed, M, H);
			ProjArgs pa = qkv_args(m, w, l, M, ad, fused);
			raw = pa.raw;
			run_gemm(m, w, pa.g, kProfGemm);
		}
		if (fused) {
			sslm_launch::AttnArgs a = attn_args(m, w, l, M);
			a.q_f = w.q_f;
			a.q_maxpart = w.mx_q;
			a.kv_f = w.kv_f;
			a.in_scale = w.normed_scale;
			a.q_site = lw.q;
			a.r_t_k = lw.r_t_k;
			a.e_t_k = lw.e_t_k;
			a.r_t_v = lw.r_t_v;
			a.e_t_v = lw.e_t_v;
			a.rope_cos = m->rope_cos;
			a.rope_sin = m->rope_sin;
			a.sat = m->sat;
			if (dbg) a.q_tap = dbg_tap(m, l, kDbgQRot);
			ProfScope p(s, kProfAttn, 0, 0);
			sslm_launch::attention_decode(a, s);
			ck(hipGetLastError());
		} else {
			sslm_launch::QkvPostArgs a{};
			a.M = M;
			a.H = H;
			a.NH = m->NH;
			a.NKV = m->NKV;
			a.D = m->D;
			a.cap = m->cap;
			a.tok = w.tok;
			a.q_f = w.q_f;
			a.q_maxpart = w.mx_q;
			a.kv_f = w.kv_f;
			a.in_scale = w.normed_scale;
			a.q_site = lw.q;
			a.r_t_k = lw.r_t_k;
			a.e_t_k = lw.e_t_k;
			a.r_t_v = lw.r_t_v;
			a.e_t_v = lw.e_t_v;
			a.rope_cos = m->rope_cos;
			a.rope_sin = m->rope_sin;
			a.block_bytes = (int64_t)m->block_bytes;
			a.layer = l;
			a.q_rot = w.q_rot;
			a.q_scale = w.q_scale;
			a.sat = m->sat;
			a.status = m->status;
			a.kv_pool = m->pool_dev;
			a.raw = raw;
			// A prefill span lands its K/V only once every token's q funnel has passed, as the
			// reference runs every q funnel of the span before the first landing
			// (forward_sites.cpp:2188-2240).
			a.kv_stage = w.kv_stage;
			a.sat_stage = w.sat_stage;
			{
				ProfScope p(s, kProfRow, 0, 0);
				sslm_launch::qkv_post(a, s);
				ck(hipGetLastError());
				if (a.kv_stage) {
					sslm_launch::kv_commit(a, s);
					ck(hipGetLastError());
				}
			}
			if (dbg) dbg_gather(m, w, l, kDbgQRot, w.q_rot, w.q_scale, nullptr, H, M);
			sslm_launch::AttnArgs aa = attn_args(m, w, l, M);
			aa.q_rot = w.q_rot;
			aa.q_scale = w.q_scale;
			ProfScope p(s, kProfAttn, 0, 0);
			sslm_launch::attention(aa, s, !decode);  // prefill chunks: one sequence, consecutive positions
			ck(hipGetLastError());
		}
		{
			sslm_launch::FunnelArgs a{};
			a.M = M;
			a.N = H;
			a.tok = w.tok;
			a.f = w.ctx_f;
			a.ld_f = H;
			a.maxpart = w.mx_ctx;
			a.ntiles = m->NH;
			a.incoming = nullptr;
			a.site = lw.ctx;
			a.out = w.ctx;
			a.out_scale = w.ctx_scale;
			a.layer = l;
			a.status = m->status;
			a.head_status = m->head_status;
			ProfScope p(s, kProfRow, 0, 0);
			sslm_launch::funnel(a, s);
			ck(hipGetLastError());
			if (dbg) dbg_gather(m, w, l, kDbgCtx, w.ctx, w.ctx_scale, nullptr, H, M);
		}
		{  // o_proj (forward_sites.cpp:1907-1914)
			const int pj[1] = {3};
			run_lora_u(m, w, ad, l, pj, 1, w.ctx, M, H);
			ProjArgs pa = o_args(m, w, l, M, ad);
			raw = pa.raw;
			run_gemm(m, w, pa.g, kProfGemm);
		}
		{  // attn residual -> mlp norm (forward_sites.cpp:1923-1936)
			sslm_launch::ResidualArgs a{};
			a.M = M;
			a.H = H;
			a.tok = w.tok;
			a.branch_f = w.o_f;
			a.branch_maxpart = w.mx_o;
			a.branch_in = w.ctx_scale;
			a.branch_site = lw.o;
			a.stream = st.codes;
			a.stream_idx = st.idx;
			a.stream_scale = st.scale;
			a.res_site = lw.attn_res;
			a.out_stream = w.attn_stream;
			a.out_idx = w.ident;
			a.out_stream_scale = w.attn_stream_scale;
			a.gain = lw.mlp_gain;
			a.norm_site = lw.mlp_norm;
			a.norm_out = w.mlp_normed;
			a.norm_scale = w.mlp_scale;
			a.norm_recip = w.mlp_recip;
			a.layer = l;
			a.status = m->status;
			a.raw = raw;
			if (dbg) a.branch_tap = dbg_tap(m, l, kDbgO);
			ProfScope p(s, kProfRow, 0, 0);
			sslm_launch::residual_norm(a, s);
			ck(hipGetLastError());
			if (dbg) {
				dbg_gather(m, w, l, kDbgAttnRes, w.attn_stream, w.attn_stream_scale, nullptr, H, M);
				dbg_gather(m, w, l, kDbgMlpNorm, w.mlp_normed, w.mlp_scale, nullptr, H, M);
			}
		}
		{  // gate | up (forward_sites.cpp:1938-1955)
			const int pj[2] = {4, 5};
			run_lora_u(m, w, ad, l, pj, 2, w.mlp_normed, M, H);
			ProjArgs pa = gu_args(m, w, l, M, ad);
			raw = pa.raw;
			run_gemm(m, w, pa.g, kProfGemm);
		}
		{
			sslm_launch::ActArgs a{};
			a.M = M;
			a.I = I;
			a.tok = w.tok;
			a.gu_f = w.gu_f;
			a.gu_maxpart = w.mx_gu;
			a.in_scale = w.mlp_scale;
			a.gate_site = lw.gate;
			a.up_site = lw.up;
			a.act_site = lw.act;
			a.silu = m->silu;
			a.act = w.act;
			a.act_scale = w.act_scale;
			a.layer = l;
			a.status = m->status;
			a.raw = raw;
			a.prod = w.act_prod;
			a.act_maxpart = w.act_maxpart;
			a.gu_scale = w.gu_scale;
			if (dbg) {
				a.gate_tap = dbg_tap(m, l, kDbgGate);
				a.up_tap = dbg_tap(m, l, kDbgUp);
			}
			ProfScope p(s, kProfRow, 0, 0);
			// decode rows: one block per (row, column slice) in two launches, instead of one
			// block per row that leaves most CUs idle
			if (decode && sslm_launch::mlp_act_sliced_ok(a)) sslm_launch::mlp_act_sliced(a, s);
			else sslm_launch::mlp_act(a, s);
			ck(hipGetLastError());
			if (dbg) dbg_gather(m, w, l, kDbgAct, w.act, w.act_scale, nullptr, I, M);
		}
		{  // down_proj (forward_sites.cpp:1969-1977)
			const int pj[1] = {6};
			run_lora_u(m, w, ad, l, pj, 1, w.act, M, I);
			ProjArgs pa = down_args(m, w, l, M, ad);
			raw = pa.raw;
			run_gemm(m, w, pa.g, kProfGemm);
		}
		{  // mlp residual -> commit -> next layer's attn norm (forward_sites.cpp:1982-2009)
			sslm_launch::ResidualArgs a{};
			a.M = M;
			a.H = H;
			a.tok = w.tok;
			a.branch_f = w.down_f;
			a.branch_maxpart = w.mx_down;
			a.branch_in = w.act_scale;
			a.branch_site = lw.down;
			a.stream = w.attn_stream;
			a.stream_idx = w.ident;
			a.stream_scale = w.attn_stream_scale;
			a.res_site = lw.mlp_res;
			a.out_stream = st.codes;
			a.out_idx = st.idx;
			a.out_stream_scale = st.scale;
			if (l + 1 < l1) {
				a.gain = m->layers[l + 1].attn_gain;
				a.norm_site = m->layers[l + 1].attn_norm;
				a.norm_out = w.normed;
				a.norm_scale = w.normed_scale;
				a.norm_recip = w.normed_recip;
			}
			a.layer = l;
			a.status = m->status;
			a.raw = raw;
			if (dbg) a.branch_tap = dbg_tap(m, l, kDbgDown);
			ProfScope p(s, kProfRow, 0, 0);
			sslm_launch::residual_norm(a, s);
			ck(hipGetLastError());
			if (dbg) dbg_gather(m, w, l, kDbgMlpRes, st.codes, st.scale, st.idx, H, M);
		}
	}
}


// final norm + LM head + lowest-index argmax for M tokens whose stream rows are st.idx
// (src/sslm_abi.cpp:2280-2289, forward_sites.cpp:2412-2441)
void run_logits(sslm_model m, Track& w, int M, StreamRef st, const TokenInfo* tok,
                const uint8_t* const* mask = nullptr) {
	hipStream_t s = w.stream;
	{
		ProfScope p(s, kProfRow, 0, 0);
		sslm_launch::RowNormArgs a{st.codes, st.idx, m->H, m->final_gain, m->final_site, w.final_codes,
		                           w.final_scale, nullptr};
		sslm_launch::rmsnorm(a, M, m->H, tok, m->status, m->L, s);
		ck(hipGetLastError());
	}
	GemmArgs g = head_args(m, w, M, tok);
	g.epi.mask_page = mask;
	run_gemm(m, w, g, kProfHead);
	sslm_launch::argmax_finalize(w.argmax_key, (m->V + 15) / 16, M, w.out_tokens, s);
	ck(hipGetLastError());
}

// Damped-greedy selection over one logit row (src/damped_greedy_topk.cpp:1-461); `page` is the
// bound schema's mask page (masked logits already INT32_MIN), null for free text.  Top-k by (logit desc, index asc); q_theta = the k i-exp values renormalized to
// Q15 (TopKRenormalizeQ15: each against the row-max peak, refused when any is out of domain);
// p_omega from the anti-LM; winner = max of q_theta - (alpha * p_omega >> 15), lowest index on
// ties.  Returns false when refused.
// The selection after top-k: `idx` and `val` are the k candidates in FsdTopK order.
bool damped_select(const int32_t* idx, const int32_t* val, const sslm_decode_params& p, const AntiLm& lm,
                   const uint8_t* page, int32_t* token) {
	const int k = p.top_k;
	auto legal = [&](int32_t t) { return !page || ((page[t >> 3] >> (t & 7)) & 1u); };
	if (check_softmax_width(p.q_b, p.q_c, k) != kOk) return false;
	int64_t row_max = val[0];
	for (int i = 1; i < k; ++i) row_max = std::max<int64_t>(row_max, val[i]);
	const int64_t peak = iexp_element(0, p.q_ln2, p.q_b, p.q_c, kI64Max);
	const bool peak_ok = peak >= 1 && peak <= kSoftmaxMaxSafe;
	std::vector<int64_t> q(k, 0);
	bool well_formed = peak_ok;
	int64_t total = 0;
	for (int i = 0; i < k; ++i) {
		const int64_t v = iexp_element((int64_t)val[i] - row_max, p.q_ln2, p.q_b, p.q_c, kI64Max);
		if (v < 0 || !peak_ok || v > peak) {  // refused construction, or outside [0, peak]
			well_formed = false;
			continue;
		}
		q[i] = v;
		total += v;
	}
	if (!well_formed) return false;
	const int64_t denom = total > 1 ? total : 1;
	for (int i = 0; i < k; ++i) q[i] = (q[i] << 15) / denom;
	std::vector<int64_t> omega(k, 0);
	lm.penalize(idx, k, omega.data());
	int64_t best = 0;
	int32_t best_tok = -1;
	for (int i = 0; i < k; ++i) {
		const int64_t score = legal(idx[i]) ? q[i] - (int32_t)(((int64_t)p.alpha_q15 * omega[i]) >> 15) : kI64Min;
		if (best_tok < 0 || score > best || (score == best && idx[i] < best_tok)) {
			best = score;
			best_tok = idx[i];
		}
	}
	*token = best_tok;
	return true;
}

// FsdTopK order: logit desc, then legal before masked, then index asc
struct TopKOrder {
	const uint8_t* page;
	bool legal(int32_t t) const { return !page || ((page[t >> 3] >> (t & 7)) & 1u); }
	bool operator()(int32_t a, int32_t va, int32_t b, int32_t vb) const {
		if (va != vb) return va > vb;
		if (legal(a) != legal(b)) return legal(a);
		return a < b;
	}
};

// Over a whole logit row (masked logits already INT32_MIN).
bool damped_pick(const int32_t* row, int V, const sslm_decode_params& p, const AntiLm& lm, const uint8_t* page,
                 int32_t* token) {
	const int k = p.top_k;
	const TopKOrder ord{page};
	std::vector<int32_t> idx(V);
	for (int i = 0; i < V; ++i) idx[i] = i;
	std::partial_sort(idx.begin(), idx.begin() + k, idx.end(),
	                  [&](int32_t a, int32_t b) { return ord(a, row[a], b, row[b]); });
	std::vector<int32_t> val(k);
	for (int i = 0; i < k; ++i) val[i] = row[idx[i]];
	return damped_select(idx.data(), val.data(), p, lm, page, token);
}

// Over the device's candidate set: the k (index, logit) pairs first in FsdTopK order, unordered.
bool damped_pick_candidates(const int2* cand, const sslm_decode_params& p, const AntiLm& lm, const uint8_t* page,
                            int32_t* token) {
	const int k = p.top_k;
	const TopKOrder ord{page};
	std::vector<int2> c(cand, cand + k);
	std::sort(c.begin(), c.end(), [&](const int2& a, const int2& b) { return ord(a.x, a.y, b.x, b.y); });
	std::vector<int32_t> idx(k), val(k);
	for (int i = 0; i < k; ++i) {
		idx[i] = c[i].x;
		val[i] = c[i].y;
	}
	return damped_select(idx.data(), val.data(), p, lm, page, token);
}

sslm_status map_forward_status(int32_t word) {
	const int32_t st = word & 0xff;
	if (st == 0) return SSLM_OK;
	if (st == kSoftmaxKernelRefusedAfterGateAccepted) return SSLM_NUMERIC_STEP_REFUSED;
	return SSLM_ARTIFACT_REJECTED;  // src/sslm_abi.cpp:1352-1360
}

// Runs an entry point's body, turning HIP errors and refused launches into statuses.  `refused`:
// the status of a launch refused by a launch wrapper (SSLM_INVALID_ARGUMENT at the boundary;
// the forward verbs pass SSLM_NUMERIC_STEP_REFUSED and leave every sequence's state as it was).
template <typename F>
sslm_status guarded(F&& f, sslm_status refused = SSLM_INVALID_ARGUMENT) {
	try {
		return f();
	} catch (const HipError& e) {
		fprintf(stderr, "sslm_hip: HIP error %d (%s)\n", (int)e.e, hipGetErrorString(e.e));
		return e.e == hipErrorOutOfMemory ? SSLM_ALLOCATION_FAILED : SSLM_INVALID_ARGUMENT;
	} catch (const std::bad_alloc&) {
		return SSLM_ALLOCATION_FAILED;
	} catch (const sslm_launch::LaunchRefused& e) {
		// nothing of the refused launch was enqueued; let what was enqueued before it finish so
		// no kernel still runs on buffers the caller may free after this status
		fprintf(stderr, "sslm_hip: launch refused (%s)\n", e.what);
		(void)hipDeviceSynchronize();
		return refused;
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
void alloc_track(sslm_model m, Track& w, int T, bool head) {
	auto& own = w.own;
	const int H = m->H, I = m->I, KVH = m->KVH;
	w.capacity = T;
	w.tok = dalloc<TokenInfo>(T, &own);
	w.tok_ids = dalloc<int32_t>(T, &own);
	w.ident = dalloc<int32_t>(T, &own);
	{
		std::vector<int32_t> id(T);
		for (int i = 0; i < T; ++i) id[i] = i;
		ck(hipMemcpy(w.ident, id.data(), T * 4, hipMemcpyHostToDevice));
	}
	w.slot_idx = dalloc<int32_t>(T, &own);
	w.out_tokens = dalloc<int32_t>(T, &own);
	w.hid_chunk = dalloc<int8_t>((size_t)T * H, &own);
	w.normed = dalloc<int8_t>((size_t)T * H, &own);
	w.q_rot = dalloc<int8_t>((size_t)T * H, &own);
	w.ctx = dalloc<int8_t>((size_t)T * H, &own);
	w.attn_stream = dalloc<int8_t>((size_t)T * H, &own);
	w.mlp_normed = dalloc<int8_t>((size_t)T * H, &own);
	w.act = dalloc<int8_t>((size_t)T * I, &own);
	w.final_codes = dalloc<int8_t>((size_t)T * H, &own);
	for (Scale** sp : {&w.hid_chunk_scale, &w.normed_scale, &w.q_scale, &w.ctx_scale, &w.attn_stream_scale,
	                   &w.mlp_scale, &w.act_scale, &w.final_scale})
		*sp = dalloc<Scale>(T, &own);
	w.normed_recip = dalloc<int64_t>(T, &own);
	w.mlp_recip = dalloc<int64_t>(T, &own);
	w.kv_f = dalloc<int64_t>((size_t)T * 2 * KVH, &own);
	w.q_f = dalloc<int32_t>((size_t)T * H, &own);
	w.ctx_f = dalloc<int32_t>((size_t)T * H, &own);
	w.o_f = dalloc<int32_t>((size_t)T * H, &own);
	w.gu_f = dalloc<int32_t>((size_t)T * 2 * I, &own);
	w.down_f = dalloc<int32_t>((size_t)T * H, &own);
	w.mx_q = dalloc<uint32_t>((size_t)(H + 2 * KVH) / 16 * kPartLd, &own);
	w.mx_ctx = dalloc<uint32_t>((size_t)m->NH * kPartLd, &own);
	w.mx_o = dalloc<uint32_t>((size_t)H / 16 * kPartLd, &own);
	w.mx_gu = dalloc<uint32_t>((size_t)2 * I / 16 * kPartLd, &own);
	w.mx_down = dalloc<uint32_t>((size_t)H / 16 * kPartLd, &own);
	w.argmax_key = head ? dalloc<unsigned long long>((size_t)(m->V + 15) / 16 * T, &own) : nullptr;
	{
		const int shapes[4][2] = {{H + 2 * KVH, H}, {H, H}, {2 * I, H}, {H, I}};
		size_t elems = 0;
		for (auto& sh : shapes) {
			for (int rows = 1; rows <= T; ++rows) {
				int sp = 1;
				const bool gemv = sslm_launch::gemv_eligible(rows, sh[1]);
				if (gemv) sp = sslm_launch::gemv_plan(rows, sh[0], sh[1], true, true).splits;
				bool narrow = false;
				if (!gemv && sslm_launch::prefill_mfma_k(sh[1])) {
					const PrefillPlan pp = sslm_launch::prefill_plan(rows, sh[0], sh[1], true);
					sp = pp.splits;
					narrow = pp.narrow;
				}
				// a GEMV and the narrow prefill kernel are always raw
				if (sp > 1 || gemv || narrow) elems = std::max(elems, (size_t)sp * rows * sh[0]);
			}
		}
		w.raw_part = elems ? dalloc<int32_t>(elems, &own) : nullptr;
	}
	for (int i = 0; i < 3; ++i) w.lora_u[i] = dalloc<int8_t>((size_t)T * kMaxRank, &own);
	w.act_prod = w.prefill ? nullptr : dalloc<int32_t>((size_t)sslm_launch::kMaxSlicedActRows * I, &own);
	w.act_maxpart = w.prefill ? nullptr : dalloc<uint32_t>((size_t)sslm_launch::kMaxActSlices * kPartLd, &own);
	w.gu_scale = w.prefill ? nullptr : dalloc<Scale>((size_t)sslm_launch::kMaxSlicedActRows * 2, &own);
	w.kv_stage = w.prefill ? dalloc<int8_t>((size_t)T * 2 * KVH, &own) : nullptr;
	w.sat_stage = w.prefill ? dalloc<uint32_t>(T, &own) : nullptr;
	// the per-token attention keeps its rows in global scratch when they exceed LDS; a prefill
	// track whose spans take the query-tiled kernel (no stored rows) needs none
	const bool rows_in_scratch = !sslm_launch::attention_in_lds(m->cap) && !(w.prefill && sslm_launch::tiled_attention_enabled());
	w.attn_scratch = rows_in_scratch ? dalloc<int64_t>((size_t)T * m->NH * m->cap, &own) : nullptr;
	w.lg_tok = head ? dalloc<TokenInfo>(T, &own) : nullptr;
	w.lg_slot = head ? dalloc<int32_t>(T, &own) : nullptr;
	w.lg_mask = head ? (const uint8_t**)dalloc<uintptr_t>(T, &own) : nullptr;
	if (!w.stream) {
		ck(hipStreamCreate(&w.stream));
		ck(hipEventCreateWithFlags(&w.done, hipEventDisableTiming));
		ck(hipEventCreateWithFlags(&w.fork, hipEventDisableTiming));
	}
	++w.gen;
}

void free_track_buffers(Track& w) {
	for (void* p : w.own) (void)hipFree(p);
	w.own.clear();
	w.capacity = 0;
}

bool packed_enabled();

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
	// A block is sized with the declared KV element width (sslm_kv_block_size,
	// src/sslm_abi.cpp:866-886), but the C ABI's layer loops store int8 rows at the start of it
	// whatever CFG1's kv_precision says (forward_sites.cpp:1227-1267; only the greedy-loop entry
	// the ABI never calls refuses Int16), so an Int16 artifact runs as int8 in a block twice the size.
	m->block_bytes = (size_t)c.layers * c.context_cap * c.kv_heads * c.head_dim * 2 * (c.kv_precision ? 2 : 1);
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
	if (A.flags & 2u) {  // damped-greedy constants (src/damped_greedy_phaseD.cpp, src/sslm_abi.cpp:1172-1185)
		if (!A.damped || A.damped_bytes != 12) {
			*err = "damped-greedy constants section missing or malformed";
			return false;
		}
		const int64_t dm = (int64_t)get64(A.damped);
		const int64_t de = (int32_t)get32(A.damped + 8);
		int64_t ql = 0, qb = 0, qc = 0;
		// in domain: the i-exp triple derives, and a softmax over the real vocabulary (151,936
		// entries) passes the row-width gate
		if (iexp_scale_constants(dm, de, m->ln2_q, m->b_q, m->ca_q, &ql, &qb, &qc) != 0 ||
		    check_softmax_width(qb, qc, 151936) != kOk) {
			*err = "damped-greedy constants out of domain";
			return false;
		}
		m->dg_available = true;
		m->dg_q_ln2 = ql;
		m->dg_q_b = qb;
		m->dg_q_c = qc;
	}
	m->page_bytes = (uint32_t)((m->V + 7) / 8);
	if (A.schemas) {  // src/sslm_abi.cpp:1193-1215
		if (!parse_schemas(A.schemas, A.schemas_bytes, (uint32_t)m->V, &m->schemas)) {
			*err = "SchemaMasks section rejected";
			return false;
		}
		m->schema_handles.resize(m->schemas.size());
		for (size_t i = 0; i < m->schemas.size(); ++i) m->schema_handles[i] = sslm_schema_s{m, (uint32_t)i};
		// the mask pages go to HBM, so masked greedy decoding takes its argmax on the device
		size_t total = 0;
		for (const SchemaEntry& e : m->schemas) {
			m->page_off.push_back(total);
			total += (size_t)e.states * m->page_bytes;
		}
		std::vector<uint8_t> pages(total);
		for (size_t i = 0; i < m->schemas.size(); ++i)
			memcpy(pages.data() + m->page_off[i], m->schemas[i].pages, (size_t)m->schemas[i].states * m->page_bytes);
		m->d_pages = dupload(pages, &own);
	}
	// Packed decode copies of every projection and the LM head (read by the decode GEMVs at
	// M <= 32; the row-major matrices stay for the prefill GEMMs).  SSLM_HIP_PACKED=0 keeps the
	// decode GEMVs on the row-major matrices.
	if (packed_enabled()) {
		auto packed = [&](const int8_t* wt, int N, int K) -> int8_t* {
			if (K % 128) return nullptr;
			int8_t* p = dalloc<int8_t>(sslm_launch::packed_bytes(N, K), &own);
			sslm_launch::pack_gemv(wt, N, K, p, nullptr);
			ck(hipGetLastError());
			return p;
		};
		for (DevLayer& d : m->layers) {
			d.p_qkv = packed(d.w_qkv, H + 2 * m->KVH, H);
			d.p_o = packed(d.w_o, H, H);
			d.p_gu = packed(d.w_gu, 2 * I, H);
			d.p_down = packed(d.w_down, H, I);
		}
		m->head_pk = packed(m->head, m->V, H);
		ck(hipDeviceSynchronize());
	}
	// slots
	m->stream_codes = dalloc<int8_t>((size_t)kSlotCapacity * H, &own);
	m->stream_scale = dalloc<Scale>(kSlotCapacity, &own);
	m->sat = dalloc<unsigned long long>(kSlotCapacity, &own);
	m->status = dalloc<int32_t>(kSlotCapacity, &own);
	m->head_status = dalloc<int32_t>(kSlotCapacity, &own);
	m->snap_codes = dalloc<int8_t>((size_t)kSlotCapacity * m->H, &own);
	m->snap_scale = dalloc<Scale>(kSlotCapacity, &own);
	m->snap_sat = dalloc<unsigned long long>(kSlotCapacity, &own);
	m->snap_kv = dalloc<int8_t>((size_t)kSlotCapacity * m->L * 2 * m->KVH, &own);
	{
		const std::vector<int32_t> none(kSlotCapacity, kHeadStatusNone);
		ck(hipMemcpy(m->head_status, none.data(), none.size() * sizeof(int32_t), hipMemcpyHostToDevice));
	}
	for (int i = kSlotCapacity - 1; i >= 0; --i) m->free_slots.push_back(i);
	// tracks: track 0 carries prefill chunks and the LM head; the others run extra token groups
	// of a decode step concurrently
	m->tracks.resize(kTracks);
	for (int i = 0; i < kTracks; ++i) alloc_track(m, m->tracks[i], i == 0 ? kMaxTokens : kTrackTokens, i == 0);
	// kernel attributes are queried and set here, outside any graph capture
	if (!sslm_launch::attention_prepare(m->D, m->NH / m->NKV)) {
		*err = "decode attention kernel attributes could not be set";
		return false;
	}
	return true;
}

// Every stream of the model: decode tracks and the prefill track.
template <typename F>
void for_each_track(sslm_model m, F&& f) {
	for (Track& w : m->tracks) f(w);
	f(m->prefill);
}

void sync_tracks(sslm_model m) {
	for_each_track(m, [](Track& w) {
		if (w.stream) ck(hipStreamSynchronize(w.stream));
	});
}

// Destroys every captured graph once no launch of one can still be in flight.
void drop_graphs(sslm_model m) {
	sync_tracks(m);
	for (auto& kv : m->graphs) (void)hipGraphExecDestroy(kv.second);
	m->graphs.clear();
	m->graph_seen.clear();
}

void free_model(sslm_model m) {
	for_each_track(m, [](Track& w) {
		if (w.stream) (void)hipStreamSynchronize(w.stream);
	});
	for (auto& kv : m->graphs) (void)hipGraphExecDestroy(kv.second);
	m->graphs.clear();
	for (void* p : m->owned) (void)hipFree(p);
	m->owned.clear();
	if (m->dbg_codes) (void)hipFree(m->dbg_codes);
	if (m->dbg_scales) (void)hipFree(m->dbg_scales);
	m->dbg_codes = nullptr;
	m->dbg_scales = nullptr;
	for_each_track(m, [](Track& w) {
		free_track_buffers(w);
		if (w.stream) (void)hipStreamDestroy(w.stream);
		if (w.done) (void)hipEventDestroy(w.done);
		if (w.fork) (void)hipEventDestroy(w.fork);
		w.stream = nullptr;
		w.done = nullptr;
		w.fork = nullptr;
	});
}

constexpr size_t kGraphCache = 64;

bool packed_enabled() {
	static const bool v = [] {
		const char* e = getenv("SSLM_HIP_PACKED");
		return !(e && e[0] == '0');
	}();
	return v;
}

bool graphs_enabled() {
	static const bool v = [] {
		const char* e = getenv("SSLM_HIP_GRAPHS");
		return !(e && atoi(e) == 0);
	}();
	return v;
}

// The captured graph for `key`, recorded from `body` on stream `s` when absent.  A full cache is
// emptied first -- after every stream has drained, since graphs launched earlier in the same
// submission may still be running.
hipGraphExec_t graph_of(sslm_model m, const std::string& key, hipStream_t s, const std::function<void()>& body) {
	auto it = m->graphs.find(key);
	if (it != m->graphs.end()) return it->second;
	if (m->graphs.size() >= kGraphCache) drop_graphs(m);
	hipGraph_t graph = nullptr;
	ck(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
	try {
		body();
	} catch (...) {
		(void)hipStreamEndCapture(s, &graph);
		if (graph) (void)hipGraphDestroy(graph);
		throw;
	}
	ck(hipStreamEndCapture(s, &graph));
	hipGraphExec_t exec = nullptr;
	const hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
	(void)hipGraphDestroy(graph);
	ck(e);
	return m->graphs.emplace(key, exec).first->second;
}
// Upload the TokenInfo of one launch sequence.
void put_tokens(Track& w, const std::vector<TokenInfo>& ti) {
	ck(hipMemcpyAsync(w.tok, ti.data(), ti.size() * sizeof(TokenInfo), hipMemcpyHostToDevice, w.stream));
}

// Tokens one prefill launch sequence takes: the whole admitted span up to kPartLd (the token
// stride of the funnels' partial maxima), unless the per-token attention must keep rows longer
// than LDS holds in global scratch (query-tiled attention switched off at a long context cap).
// SSLM_HIP_PREFILL_SPAN (read per call; tests use it) lowers the limit, forcing several spans.
int prefill_limit(sslm_model m) {
	int lim = (sslm_launch::attention_in_lds(m->cap) || sslm_launch::tiled_attention_enabled()) ? kPartLd : kMaxTokens;
	const char* e = getenv("SSLM_HIP_PREFILL_SPAN");
	if (e && atoi(e) > 0) lim = std::min(lim, atoi(e));
	return lim;
}

// The prefill track with room for T tokens (grown in steps of kMaxTokens; graphs that captured
// the old buffers are dropped first).
Track& prefill_track(sslm_model m, int T) {
	Track& w = m->prefill;
	if (w.capacity >= T) return w;
	drop_graphs(m);
	free_track_buffers(w);
	w.prefill = true;
	alloc_track(m, w, (T + kMaxTokens - 1) / kMaxTokens * kMaxTokens, false);
	return w;
}

// Prefill of `n` admitted tokens (PrefillWholeTokensImpl, src/sslm_abi.cpp:1481-1545).  The
// reference embeds every admitted token, then runs one batched layer loop over all of them, and
// commits nothing when any step refuses.  Here the span is one launch sequence (embed, then every
// layer site over all its tokens) when it fits prefill_limit(), else consecutive spans of that
// many tokens; the sequence's state (stream row, context length) is committed once, after every
// span has passed.  A repeated span shape replays a captured graph.
sslm_status prefill_tokens(sslm_model m, sslm_seq s, const int32_t* tokens, int n) {
	m->pool_dev = s->pool->dev;
	const int P = prefill_limit(m);
	Track& w = prefill_track(m, std::min(n, P));
	const int H = m->H;
	std::deque<std::vector<TokenInfo>> staged;  // host copies stay alive until the sync below
	int done = 0;
	int last_T = 0;
	// Several spans land K/V rows and clamp counts span by span, before a later span can refuse;
	// the reference runs the whole call as one batch.  The call's rows [ctx, ctx + n) of every
	// layer's K and V and the slot's clamp counter are saved first and put back on a refusal, which
	// reproduces the reference exactly for refusals before its first landing (embedding, layer 0
	// RMSNorm and q funnel); for a refusal at a later layer the reference keeps the landings it made,
	// which no later call reads (positions past the committed context) but a blob or KV peek shows.
	const bool multi = n > P;
	int8_t* kv_save = nullptr;
	unsigned long long* sat_save = nullptr;
	const size_t run = (size_t)n * m->D, runs = (size_t)m->L * 2 * m->NKV, pitch = (size_t)m->cap * m->D;
	int8_t* const block = s->pool->dev + (size_t)s->block * s->pool->block_size + (size_t)s->context_length * m->D;
	if (multi) {
		ck(hipMalloc(&kv_save, run * runs + 64));
		sat_save = (unsigned long long*)(kv_save + ((run * runs + 7) & ~(size_t)7));
		ck(hipMemcpy2DAsync(kv_save, run, block, pitch, run, runs, hipMemcpyDeviceToDevice, w.stream));
		ck(hipMemcpyAsync(sat_save, m->sat + s->slot, 8, hipMemcpyDeviceToDevice, w.stream));
	}
	struct SaveGuard {
		int8_t* p;
		~SaveGuard() {
			if (p) (void)hipFree(p);
		}
	} save_guard{kv_save};
	while (done < n) {
		const int T = std::min(P, n - done);
		staged.emplace_back(T);
		std::vector<TokenInfo>& ti = staged.back();
		for (int t = 0; t < T; ++t) ti[t] = TokenInfo{s->context_length + done + t, s->slot, (int32_t)s->block};
		ck(hipMemcpyAsync(w.tok, ti.data(), T * sizeof(TokenInfo), hipMemcpyHostToDevice, w.stream));
		ck(hipMemcpyAsync(w.tok_ids, tokens + done, T * 4, hipMemcpyHostToDevice, w.stream));
		auto body = [&]() {
			{
				ProfScope p(w.stream, kProfRow, 0, 0);
				sslm_launch::embed(w.tok_ids, T, m->embed, H, m->V, m->embed_site, w.hid_chunk, w.ident,
				                   w.hid_chunk_scale, w.ident, w.tok, m->status, w.stream);
				ck(hipGetLastError());
			}
			run_layers(m, w, T, StreamRef{w.hid_chunk, w.hid_chunk_scale, w.ident}, 0, m->L, s->adapter, false);
		};
		const std::string key = "p|" + std::to_string(T) + "|" + std::to_string((uintptr_t)s->adapter) + "|" +
		                        std::to_string((uintptr_t)m->pool_dev) + "|" + std::to_string(w.gen);
		// a span shape is captured the second time it is seen: one-off shapes launch directly
		try {
			if (graphs_enabled() && !prof_enabled() && !m->dbg_codes && m->graph_seen[key]++ > 0)
				ck(hipGraphLaunch(graph_of(m, key, w.stream, body), w.stream));
			else
				body();
		} catch (const sslm_launch::LaunchRefused&) {
			// nothing is committed; clear what the enqueued kernels reported for the slot
			ck(hipStreamSynchronize(w.stream));
			ck(hipMemset(m->status + s->slot, 0, 4));
			throw;
		}
		done += T;
		last_T = T;
	}
	int32_t word = 0;
	ck(hipMemcpyAsync(&word, m->status + s->slot, 4, hipMemcpyDeviceToHost, w.stream));
	ck(hipStreamSynchronize(w.stream));
	prof_collect();
	if (word != 0) {
		ck(hipMemset(m->status + s->slot, 0, 4));
		if (multi) {
			ck(hipMemcpy2DAsync(block, pitch, kv_save, run, run, runs, hipMemcpyDeviceToDevice, w.stream));
			ck(hipMemcpyAsync(m->sat + s->slot, sat_save, 8, hipMemcpyDeviceToDevice, w.stream));
			ck(hipStreamSynchronize(w.stream));
		}
		return map_forward_status(word);
	}
	// the span's last row becomes the sequence's stream state
	ck(hipMemcpyAsync(m->stream_codes + (size_t)s->slot * H, w.hid_chunk + (size_t)(last_T - 1) * H, H,
	                  hipMemcpyDeviceToDevice, w.stream));
	ck(hipMemcpyAsync(m->stream_scale + s->slot, w.hid_chunk_scale + (last_T - 1), sizeof(Scale),
	                  hipMemcpyDeviceToDevice, w.stream));
	ck(hipStreamSynchronize(w.stream));
	s->context_length += n;
	s->layer_index = 0;
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
	{
		std::lock_guard<std::mutex> lk(pool->model->mu);
		for_each_track(pool->model, [](Track& w) {
			if (w.stream) (void)hipStreamSynchronize(w.stream);
		});
	}
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
		ck(hipMemsetAsync(p->dev + (size_t)block * p->block_size, 0, p->block_size, model->tracks[0].stream));
		ck(hipMemsetAsync(model->stream_codes + (size_t)slot * model->H, 0, model->H, model->tracks[0].stream));
		ck(hipMemsetAsync(model->stream_scale + slot, 0, sizeof(Scale), model->tracks[0].stream));
		ck(hipMemsetAsync(model->sat + slot, 0, 8, model->tracks[0].stream));
		ck(hipMemsetAsync(model->status + slot, 0, 4, model->tracks[0].stream));
		ck(hipStreamSynchronize(model->tracks[0].stream));
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
		                  m->tracks[0].stream));
		ck(hipMemsetAsync(m->stream_codes + (size_t)seq->slot * m->H, 0, m->H, m->tracks[0].stream));
		ck(hipMemsetAsync(m->stream_scale + seq->slot, 0, sizeof(Scale), m->tracks[0].stream));
		ck(hipMemsetAsync(m->sat + seq->slot, 0, 8, m->tracks[0].stream));
		ck(hipStreamSynchronize(m->tracks[0].stream));
		seq->context_length = 0;
		seq->layer_index = 0;
		seq->current_token = -1;
		seq->ready_for_logits = false;
		seq->forced_token_count = 0;
		seq->anti_lm.reset(0);
		seq->walk = seq->schema ? 0u : kWalkUnused;
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
	if (kind == SSLM_SPAN_SCHEMA_CONTENT && !seq->schema) return SSLM_SCHEMA_SPAN_UNBOUND;
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
		const int32_t admit_idcap = std::min(admit_id, admit_cap);
		// a schema-content span walks the bound schema's DFA; the first token without a
		// transition ends the admitted prefix (src/sslm_abi.cpp:1480-1510)
		const SchemaEntry* se = kind == SSLM_SPAN_SCHEMA_CONTENT ? &model->schemas[seq->schema->index] : nullptr;
		int32_t admit = admit_idcap;
		uint32_t walk_after = seq->walk;
		if (se) {
			uint32_t w = seq->walk;
			for (int32_t i = 0; i < admit_idcap; ++i) {
				uint32_t nx = 0;
				if (!schema_next(*se, w, (uint32_t)tokens[i], &nx)) {
					admit = i;
					break;
				}
				w = nx;
			}
			walk_after = w;
		}
		sslm_status stop = SSLM_OK;
		if (admit < n) {
			if (admit < admit_idcap) stop = SSLM_SCHEMA_SPAN_UNREACHABLE;
			else stop = admit_id <= admit_cap ? SSLM_TOKEN_ID_OUT_OF_RANGE : SSLM_CONTEXT_CAP_EXCEEDED;
		}
		if (admit > 0) {
			const sslm_status st = prefill_tokens(model, seq, tokens, admit);
			if (st != SSLM_OK) return st;
			if (se) {
				seq->walk = walk_after;
				seq->forced_token_count += admit;
			}
			seq->current_token = tokens[admit - 1];
			*consumed = admit;
			seq->ready_for_logits = true;  // src/sslm_abi.cpp:1969-1972
		}
		return stop;
	}, SSLM_NUMERIC_STEP_REFUSED);
}

sslm_launch::SlotCopyArgs slot_copy_args(sslm_model m, const TokenInfo* tok, int l0, int l1) {
	sslm_launch::SlotCopyArgs a{};
	a.tok = tok;
	a.codes = m->stream_codes;
	a.scale = m->stream_scale;
	a.sat = m->sat;
	a.snap_codes = m->snap_codes;
	a.snap_scale = m->snap_scale;
	a.snap_sat = m->snap_sat;
	a.kv_pool = m->pool_dev;
	a.block_bytes = (int64_t)m->block_bytes;
	a.cap = m->cap;
	a.H = m->H;
	a.NKV = m->NKV;
	a.D = m->D;
	a.l0 = l0;
	a.l1 = l1;
	a.snap_kv = m->snap_kv;
	a.snap_kv_ld = (int64_t)m->L * 2 * m->KVH;
	return a;
}

// Decode tokens are independent, so a batch's layer work can be dealt to up to kTracks streams
// as token groups of at least track_min() tokens each, so that one group's latency-bound row
// kernels could overlap another's GEMVs.  Measured on MI355X this is slower than one group (the
// groups' kernels do not overlap usefully), so one track is the default and SSLM_HIP_TRACKS
// opts in.  Everything -- embeds, layers, the joined LM head and the status read-back -- is one
// submission with one host sync.

int track_limit() {
	static const int v = [] {
		const char* e = getenv("SSLM_HIP_TRACKS");
		const int x = e ? atoi(e) : 1;
		return std::max(1, std::min(kTracks, x));
	}();
	return v;
}
int track_min() {
	static const int v = [] {
		const char* e = getenv("SSLM_HIP_TRACK_MIN_TOKENS");
		return std::max(1, e ? atoi(e) : 4);
	}();
	return v;
}

static sslm_status decode_batch(sslm_model m, sslm_seq* seqs, int32_t n, const sslm_decode_params& params,
                                int32_t* out_tokens, sslm_status* stop) {
	const uint32_t budget = (uint32_t)params.layer_budget;
	const bool damped = params.mode == SSLM_DECODE_MODE_DAMPED_GREEDY;
	// Partition: sequences needing layers, grouped by their current layer; sequences needing logits.
	std::vector<int> need_logits;
	std::vector<std::pair<uint32_t, std::vector<int>>> groups;
	for (int i = 0; i < n; ++i) {
		sslm_seq s = seqs[i];
		if (s->ready_for_logits) {
			need_logits.push_back(i);
			continue;
		}
		if (s->layer_index == 0 && s->context_length >= m->cap) {  // src/sslm_abi.cpp:2233-2236
			*stop = SSLM_CONTEXT_CAP_EXCEEDED;
			out_tokens[i] = -1;
			n = i;
			break;
		}
		if (s->layer_index >= (uint32_t)m->L) {
			// a whole token whose schema walk had no transition (-2) rests at the last layer; the
			// reference's layer loop then refuses the next call (its layer_index < L guard), mapped
			// to SSLM_ARTIFACT_REJECTED, after the sequences before it in the call
			*stop = SSLM_ARTIFACT_REJECTED;
			n = i;
			break;
		}
		auto it = std::find_if(groups.begin(), groups.end(), [&](auto& g) { return g.first == s->layer_index; });
		if (it == groups.end()) groups.push_back({s->layer_index, {i}});
		else it->second.push_back(i);
	}
	need_logits.erase(std::remove_if(need_logits.begin(), need_logits.end(), [&](int i) { return i >= n; }),
	                  need_logits.end());

	// launch units: (layer range, adapter, tokens), at most kTrackTokens tokens each
	struct Unit {
		uint32_t l0, l1;
		sslm_adapter ad;
		std::vector<int> idx;
	};
	std::vector<Unit> units;
	std::vector<int> finished;
	for (auto& g : groups) {
		const uint32_t l0 = g.first;
		const uint32_t l1 = std::min<uint32_t>(m->L, l0 + budget);
		std::vector<sslm_adapter> ads;
		for (int i : g.second)
			if (std::find(ads.begin(), ads.end(), seqs[i]->adapter) == ads.end()) ads.push_back(seqs[i]->adapter);
		for (sslm_adapter ad : ads) {
			std::vector<int> members;
			for (int i : g.second)
				if (seqs[i]->adapter == ad) members.push_back(i);
			const int total = (int)members.size();
			int parts = std::max(1, std::min(track_limit(), total / track_min()));
			parts = std::max(parts, (total + kTrackTokens - 1) / kTrackTokens);
			for (int p = 0; p < parts; ++p) {
				const int b = (int)((int64_t)total * p / parts), e = (int)((int64_t)total * (p + 1) / parts);
				if (e > b) units.push_back(Unit{l0, l1, ad, std::vector<int>(members.begin() + b, members.begin() + e)});
			}
		}
		if (l1 == (uint32_t)m->L)
			for (int i : g.second) finished.push_back(i);
	}
	std::vector<int> lg = need_logits;
	lg.insert(lg.end(), finished.begin(), finished.end());
	// whole logit rows come back to the host for damped greedy; a schema-bound sequence's greedy
	// argmax is masked on the device (its mask page per token)
	// Damped greedy takes the head's raw int32 rows; up to kTopKMax candidates per row are chosen
	// on the device and only they come back, else the whole rows do.
	const bool cands = damped && params.top_k <= sslm_launch::kTopKMax;
	const bool rows_needed = damped && !cands;
	bool masked = false;
	for (int i : lg) masked = masked || seqs[i]->schema;
	if (damped && !m->logits) m->logits = dalloc<int32_t>((size_t)kMaxTokens * m->V, &m->owned);
	if (cands && !m->topk) m->topk = dalloc<int2>((size_t)kMaxTokens * sslm_launch::kTopKMax, &m->owned);

	// Host staging, uploaded before the kernels (kept alive until the sync below).  The common
	// shape -- at most one unit per track and one head chunk -- stages every unit's tokens in its
	// track's own buffers up front and replays a captured graph of the whole submission;
	// anything else launches directly, uploading as it goes.
	Track& t0 = m->tracks[0];
	const size_t ntr = m->tracks.size();
	const bool one_per_track = units.size() <= ntr && lg.size() <= (size_t)kMaxTokens;
	const bool use_graph = one_per_track && graphs_enabled() && !prof_enabled() && !m->dbg_codes;
	std::deque<std::vector<TokenInfo>> h_tok;  // deque: references to earlier entries stay valid
	std::deque<std::vector<int32_t>> h_i32;
	std::deque<std::vector<const uint8_t*>> h_ptr;
	// the grouped decode attention's score rows for a unit: from its widest row (pos + 1)
	auto unit_wcap = [&](const Unit& un) {
		int64_t mw = 1;
		for (int i : un.idx) mw = std::max<int64_t>(mw, (int64_t)seqs[i]->context_length + 1);
		return sslm_launch::group_width_cap(mw, m->cap);
	};
	auto stage_unit = [&](size_t u, hipStream_t s) {
		const Unit& un = units[u];
		Track& w = m->tracks[u % ntr];
		const int M = (int)un.idx.size();
		w.attn_wcap = unit_wcap(un);
		h_tok.emplace_back(M);
		std::vector<TokenInfo>& ti = h_tok.back();
		h_i32.emplace_back(M);
		std::vector<int32_t>& slots = h_i32.back();
		h_i32.emplace_back(M);
		std::vector<int32_t>& ids = h_i32.back();
		for (int t = 0; t < M; ++t) {
			sslm_seq q = seqs[un.idx[t]];
			ti[t] = TokenInfo{q->context_length, q->slot, (int32_t)q->block};
			slots[t] = q->slot;
			ids[t] = q->current_token;
		}
		ck(hipMemcpyAsync(w.tok, ti.data(), M * sizeof(TokenInfo), hipMemcpyHostToDevice, s));
		ck(hipMemcpyAsync(w.slot_idx, slots.data(), M * 4, hipMemcpyHostToDevice, s));
		if (un.l0 == 0) ck(hipMemcpyAsync(w.tok_ids, ids.data(), M * 4, hipMemcpyHostToDevice, s));
	};
	// units whose snapshot was enqueued for execution (not merely recorded into a graph that a
	// refused launch then discarded): what a refused launch must restore
	std::vector<char> snapped(units.size(), 0);
	bool capturing = false;
	auto launch_unit = [&](size_t u) {
		const Unit& un = units[u];
		Track& w = m->tracks[u % ntr];
		const int M = (int)un.idx.size();
		w.attn_wcap = unit_wcap(un);
		// snapshot of the rows this unit changes, restored if an earlier sequence of the call refuses
		sslm_launch::slot_state_copy(slot_copy_args(m, w.tok, (int)un.l0, (int)un.l1), M, false, w.stream);
		ck(hipGetLastError());
		if (!capturing) snapped[u] = 1;
		if (un.l0 == 0) {  // embed the pending token (src/sslm_abi.cpp:2237-2249)
			ProfScope p(w.stream, kProfRow, 0, 0);
			sslm_launch::embed(w.tok_ids, M, m->embed, m->H, m->V, m->embed_site, m->stream_codes, w.slot_idx,
			                   m->stream_scale, w.slot_idx, w.tok, m->status, w.stream);
			ck(hipGetLastError());
		}
		run_layers(m, w, M, StreamRef{m->stream_codes, m->stream_scale, w.slot_idx}, (int)un.l0, (int)un.l1, un.ad, true);
	};
	auto stage_logits = [&](size_t b, int M, hipStream_t s) {
		h_tok.emplace_back(M);
		std::vector<TokenInfo>& ti = h_tok.back();
		h_i32.emplace_back(M);
		std::vector<int32_t>& slots = h_i32.back();
		for (int t = 0; t < M; ++t) {
			sslm_seq q = seqs[lg[b + t]];
			ti[t] = TokenInfo{q->context_length, q->slot, (int32_t)q->block};
			slots[t] = q->slot;
		}
		ck(hipMemcpyAsync(t0.lg_tok, ti.data(), M * sizeof(TokenInfo), hipMemcpyHostToDevice, s));
		ck(hipMemcpyAsync(t0.lg_slot, slots.data(), M * 4, hipMemcpyHostToDevice, s));
		if (masked) {
			h_ptr.emplace_back(M, nullptr);
			std::vector<const uint8_t*>& pg = h_ptr.back();
			for (int t = 0; t < M; ++t) {
				sslm_seq q = seqs[lg[b + t]];
				if (q->schema)
					pg[t] = m->d_pages + m->page_off[q->schema->index] + (size_t)q->walk * m->page_bytes;
			}
			ck(hipMemcpyAsync(t0.lg_mask, pg.data(), M * sizeof(void*), hipMemcpyHostToDevice, s));
		}
	};
	auto launch_logits = [&](int M) {
		run_logits(m, t0, M, StreamRef{m->stream_codes, m->stream_scale, t0.lg_slot}, t0.lg_tok,
		           masked ? t0.lg_mask : nullptr);
		if (damped) {  // the whole logit rows as well: the head's raw int32 accumulators
			GemmArgs g = head_args(m, t0, M, t0.lg_tok);
			g.epi.argmax_key = nullptr;
			g.epi.raw_out = m->logits;
			run_gemm(m, t0, g, kProfHead);
			if (cands) {
				sslm_launch::topk_candidates(m->logits, m->V, M, masked ? t0.lg_mask : nullptr, params.top_k, m->topk,
				                             t0.stream);
				ck(hipGetLastError());
			}
		}
	};
	std::vector<int32_t> rows(rows_needed ? lg.size() * (size_t)m->V : 0);
	std::vector<int2> cand(cands ? lg.size() * (size_t)params.top_k : 0);
	// every sequence of one call shares the pool of the first (checked by the caller)
	m->pool_dev = seqs[0]->pool->dev;
	std::vector<int32_t> toks(lg.size());
	try {
		if (one_per_track) {
			for (size_t u = 0; u < units.size(); ++u) stage_unit(u, t0.stream);
			if (!lg.empty()) stage_logits(0, (int)lg.size(), t0.stream);
			// Each unit is its own captured graph on its own track's stream (a graph runs its nodes
			// in order on the stream it is launched on, so one graph per track keeps the tracks
			// concurrent), forked from and joined back into track 0; the head is one more graph.
			const size_t nt = std::min(ntr, units.size());
			ck(hipEventRecord(t0.fork, t0.stream));
			for (size_t k = 1; k < nt; ++k) ck(hipStreamWaitEvent(m->tracks[k].stream, t0.fork, 0));
			for (size_t u = 0; u < units.size(); ++u) {
				Track& w = m->tracks[u % ntr];
				if (use_graph) {
					const Unit& un = units[u];
					const std::string key = "u" + std::to_string(u % ntr) + "|" + std::to_string(un.idx.size()) + "|" +
					                        std::to_string(un.l0) + "|" + std::to_string(un.l1) + "|" +
					                        std::to_string((uintptr_t)un.ad) + "|" + std::to_string((uintptr_t)m->pool_dev) +
					                        (sslm_launch::grouped_attention_chosen((int)un.idx.size(), m->NKV, m->cap)
					                             ? "|g" + std::to_string(unit_wcap(un)) + "h" +
					                                   std::to_string(sslm_launch::group_row_halves(
					                                       (int)un.idx.size(), m->NKV, m->NH / m->NKV))
					                             : "");
					capturing = true;
					const hipGraphExec_t ge = graph_of(m, key, w.stream, [&] { launch_unit(u); });
					capturing = false;
					ck(hipGraphLaunch(ge, w.stream));
					snapped[u] = 1;
				} else {
					launch_unit(u);
				}
			}
			for (size_t k = 1; k < nt; ++k) {
				ck(hipEventRecord(m->tracks[k].done, m->tracks[k].stream));
				ck(hipStreamWaitEvent(t0.stream, m->tracks[k].done, 0));
			}
			if (!lg.empty()) {
				const int M = (int)lg.size();
				if (use_graph)
					ck(hipGraphLaunch(graph_of(m, "lg|" + std::to_string(M) + (rows_needed ? "|r" : "") +
					                                  (cands ? "|c" + std::to_string(params.top_k) : "") + (masked ? "|m" : ""),
					                           t0.stream,
					                           [&] { launch_logits(M); }),
					                  t0.stream));
				else launch_logits(M);
			}
			if (!lg.empty()) ck(hipMemcpyAsync(toks.data(), t0.out_tokens, lg.size() * 4, hipMemcpyDeviceToHost, t0.stream));
			if (rows_needed && !lg.empty())
				ck(hipMemcpyAsync(rows.data(), m->logits, rows.size() * 4, hipMemcpyDeviceToHost, t0.stream));
			if (cands && !lg.empty())
				ck(hipMemcpyAsync(cand.data(), m->topk, cand.size() * sizeof(int2), hipMemcpyDeviceToHost, t0.stream));
		} else {
			std::vector<bool> used(ntr, false);
			for (size_t u = 0; u < units.size(); ++u) {
				stage_unit(u, m->tracks[u % ntr].stream);
				used[u % ntr] = true;
				launch_unit(u);
			}
			for (size_t k = 1; k < ntr; ++k) {
				if (!used[k]) continue;
				ck(hipEventRecord(m->tracks[k].done, m->tracks[k].stream));
				ck(hipStreamWaitEvent(t0.stream, m->tracks[k].done, 0));
			}
			for (size_t b = 0; b < lg.size(); b += kMaxTokens) {
				const int M = (int)std::min(lg.size() - b, (size_t)kMaxTokens);
				stage_logits(b, M, t0.stream);
				launch_logits(M);
				ck(hipMemcpyAsync(toks.data() + b, t0.out_tokens, M * 4, hipMemcpyDeviceToHost, t0.stream));
				if (rows_needed)
					ck(hipMemcpyAsync(rows.data() + b * (size_t)m->V, m->logits, (size_t)M * m->V * 4, hipMemcpyDeviceToHost,
					                  t0.stream));
				if (cands)
					ck(hipMemcpyAsync(cand.data() + b * (size_t)params.top_k, m->topk, (size_t)M * params.top_k * sizeof(int2),
					                  hipMemcpyDeviceToHost, t0.stream));
			}
		}
	} catch (const sslm_launch::LaunchRefused&) {
		// A launch wrapper refused a launch before enqueuing it.  Let what was enqueued finish,
		// put back the rows of every unit that ran (or began to run) from its snapshot and clear
		// the call's status words: the host state of every sequence was not advanced, so the call
		// leaves the sequences as it found them.
		ck(hipDeviceSynchronize());
		for (size_t u = 0; u < units.size(); ++u) {
			if (!snapped[u]) continue;
			std::vector<TokenInfo> back;
			for (int i : units[u].idx) back.push_back(TokenInfo{seqs[i]->context_length, seqs[i]->slot, (int32_t)seqs[i]->block});
			ck(hipMemcpy(t0.tok, back.data(), back.size() * sizeof(TokenInfo), hipMemcpyHostToDevice));
			sslm_launch::slot_state_copy(slot_copy_args(m, t0.tok, (int)units[u].l0, (int)units[u].l1), (int)back.size(),
			                             true, t0.stream);
			ck(hipGetLastError());
			ck(hipStreamSynchronize(t0.stream));
		}
		for (int i = 0; i < n; ++i) ck(hipMemset(m->status + seqs[i]->slot, 0, 4));
		throw;
	}
	std::vector<int32_t> words(kSlotCapacity);
	ck(hipMemcpyAsync(words.data(), m->status, kSlotCapacity * 4, hipMemcpyDeviceToHost, t0.stream));
	ck(hipStreamSynchronize(t0.stream));
	prof_collect();

	// Outcomes in call order.  The reference runs the sequences one after another and returns at
	// the first refusal (src/sslm_abi.cpp:2213-2430): the refusing sequence keeps its last
	// commit (a layer failure leaves it at the failing layer; a head failure after its layers
	// at layer L with the context advanced), its output entry and every later sequence are left
	// as they were.  The batch ran every sequence at once, so a later sequence's device stream
	// row, scale and clamp counter, and the K/V rows its unit's layers landed at its position, are
	// restored from the snapshot its unit took.  Layer failures carry their layer in the
	// status word, head failures the layer count.
	std::vector<int> in_lg(n, -1);
	for (size_t k = 0; k < lg.size(); ++k) in_lg[lg[k]] = (int)k;
	std::vector<uint32_t> unit_l1(n, 0);
	std::vector<char> in_unit(n, 0);
	for (auto& g : groups)
		for (int i : g.second) {
			unit_l1[i] = std::min<uint32_t>(m->L, g.first + budget);
			in_unit[i] = 1;
		}
	for (int i = 0; i < n; ++i)
		if (words[seqs[i]->slot] != 0) ck(hipMemsetAsync(m->status + seqs[i]->slot, 0, 4, t0.stream));
	sslm_status first_err = SSLM_OK;
	int stop_at = n;  // sequences from here on are left untouched
	for (int i = 0; i < n && stop_at == n; ++i) {
		sslm_seq s = seqs[i];
		const int32_t w = words[s->slot];
		if (w != 0 && (w >> 8) < m->L) {  // a layer refused: the last commit is the layer before it
			s->layer_index = (uint32_t)(w >> 8);
			first_err = map_forward_status(w);
			stop_at = i + 1;
			break;
		}
		if (in_unit[i]) {
			s->layer_index = unit_l1[i];
			if (unit_l1[i] < (uint32_t)m->L) out_tokens[i] = -1;
			else s->context_length += 1;
		}
		const int k = in_lg[i];
		if (k < 0) continue;
		s->ready_for_logits = false;
		if (w != 0) {  // final norm or logits refused
			first_err = map_forward_status(w);
			stop_at = i + 1;
			break;
		}
		int32_t tok = toks[k];
		const SchemaEntry* se = s->schema ? &m->schemas[s->schema->index] : nullptr;
		const uint8_t* page = se ? se->pages + (size_t)s->walk * m->page_bytes : nullptr;
		int32_t* row = rows_needed ? rows.data() + k * (size_t)m->V : nullptr;
		if (se && row)  // damped: the mask first, masked logits INT32_MIN (forward_sites.cpp:2443-2449)
			for (int t = 0; t < m->V; ++t)
				if (!((page[t >> 3] >> (t & 7)) & 1u)) row[t] = INT32_MIN;
		if (damped) {  // src/sslm_abi.cpp:2301-2384
			if (s->anti_lm.order == 0 || s->anti_lm.order != params.anti_lm_max_order)
				s->anti_lm.reset(params.anti_lm_max_order);
			const bool ok = cands ? damped_pick_candidates(cand.data() + k * (size_t)params.top_k, params, s->anti_lm, page, &tok)
			                      : damped_pick(row, m->V, params, s->anti_lm, page, &tok);
			if (!ok) {
				first_err = map_forward_status(kSoftmaxKernelRefusedAfterGateAccepted);
				stop_at = i + 1;
				break;
			}
		}  // greedy: tok is the device's argmax, masked for a schema-bound sequence
		if (se) {  // the walk advances only along an existing transition; none is a dead end (-2)
			uint32_t nx = 0;
			if (!schema_next(*se, s->walk, (uint32_t)tok, &nx)) {
				out_tokens[i] = -2;
				continue;
			}
			s->walk = nx;
		}
		if (damped) s->anti_lm.update(tok);
		s->current_token = tok;
		s->layer_index = 0;
		out_tokens[i] = tok;
	}
	for (auto& g : groups) {  // one restore per layer range
		std::vector<TokenInfo> restore;
		for (int i : g.second)
			if (i >= stop_at) restore.push_back(TokenInfo{seqs[i]->context_length, seqs[i]->slot, (int32_t)seqs[i]->block});
		if (restore.empty()) continue;
		ck(hipMemcpyAsync(t0.tok, restore.data(), restore.size() * sizeof(TokenInfo), hipMemcpyHostToDevice, t0.stream));
		sslm_launch::slot_state_copy(slot_copy_args(m, t0.tok, (int)g.first, (int)unit_l1[g.second[0]]), (int)restore.size(),
		                             true, t0.stream);
		ck(hipGetLastError());
		ck(hipStreamSynchronize(t0.stream));
	}
	ck(hipStreamSynchronize(t0.stream));
	return first_err;
}

static sslm_status decode_impl(sslm_model model, sslm_seq* seqs, int32_t n, const sslm_decode_params* params,
                               int32_t* out_tokens) {
	if (!model || !seqs || !params || !out_tokens) return SSLM_INVALID_ARGUMENT;
	if (n < 1) return SSLM_INVALID_ARGUMENT;
	if (params->struct_size != sizeof(sslm_decode_params)) return SSLM_INVALID_ARGUMENT;
	if (params->layer_budget < 1 || params->layer_budget > model->L) return SSLM_INVALID_ARGUMENT;
	// src/sslm_abi.cpp:2004-2035: the mode and, for damped greedy, alpha in [0, 2^20), anti-LM
	// order >= 1, 1 <= top_k <= vocab, the artifact's constants, the top-k softmax width and a
	// constructible i-exp peak
	if (params->mode != SSLM_DECODE_MODE_GREEDY && params->mode != SSLM_DECODE_MODE_DAMPED_GREEDY)
		return SSLM_INVALID_ARGUMENT;
	if (params->mode == SSLM_DECODE_MODE_DAMPED_GREEDY) {
		if (params->alpha_q15 < 0 || params->alpha_q15 >= (1 << 20) || params->anti_lm_max_order < 1 ||
		    params->top_k < 1 || params->top_k > model->V)
			return SSLM_INVALID_ARGUMENT;
		if (!model->dg_available) return SSLM_ARTIFACT_REJECTED;
		if (check_softmax_width(params->q_b, params->q_c, params->top_k) != kOk) return SSLM_INVALID_ARGUMENT;
		if (params->q_ln2 < 1 || params->q_ln2 > kI64Max / 30) return SSLM_INVALID_ARGUMENT;  // the peak's construction
	}
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
			// entries the call never reaches keep the caller's values, as in the reference
			constexpr int32_t kUntouched = INT32_MIN;
			std::vector<int32_t> out(run.size(), kUntouched);
			sslm_status stop = SSLM_OK;
			const sslm_status st = decode_batch(model, run.data(), (int32_t)run.size(), *params, out.data(), &stop);
			for (size_t k = 0; k < run.size(); ++k)
				if (out[k] != kUntouched) out_tokens[idx[k]] = out[k];
			if (st != SSLM_OK) return st;
			if (stop != SSLM_OK) return stop;
			i = j;
		}
		return SSLM_OK;
	}, SSLM_NUMERIC_STEP_REFUSED);
}

// src/sslm_abi.cpp:2436-2449: the v1.1 verb reads only the layer budget (its struct was one
// int32_t) and decodes greedily; sslm_decode_step_v2 takes the whole struct.
sslm_status sslm_decode_step(sslm_model model, sslm_seq* seqs, int32_t n, const sslm_decode_params* params,
                             sslm_workspace ws, int32_t* out_tokens) {
	(void)ws;
	if (!params) return SSLM_INVALID_ARGUMENT;
	sslm_decode_params legacy{};
	legacy.layer_budget = params->layer_budget;
	legacy.struct_size = sizeof(legacy);
	legacy.mode = SSLM_DECODE_MODE_GREEDY;
	return decode_impl(model, seqs, n, &legacy, out_tokens);
}

sslm_status sslm_decode_step_v2(sslm_model model, sslm_seq* seqs, int32_t n, const sslm_decode_params* params,
                                sslm_workspace ws, int32_t* out_tokens) {
	(void)ws;
	return decode_impl(model, seqs, n, params, out_tokens);
}

sslm_status sslm_decode_params_init(sslm_model model, int32_t mode, int32_t layer_budget, sslm_decode_params* out) {
	if (!model || !out || layer_budget < 1 || layer_budget > model->L) return SSLM_INVALID_ARGUMENT;
	if (mode != SSLM_DECODE_MODE_GREEDY && mode != SSLM_DECODE_MODE_DAMPED_GREEDY) return SSLM_INVALID_ARGUMENT;
	sslm_decode_params p{};
	p.layer_budget = layer_budget;
	p.struct_size = sizeof(p);
	p.mode = mode;
	if (mode == SSLM_DECODE_MODE_DAMPED_GREEDY) {  // src/sslm_abi.cpp:2473-2484
		if (!model->dg_available) return SSLM_ARTIFACT_REJECTED;
		p.alpha_q15 = SSLM_DAMPED_GREEDY_DEFAULT_ALPHA_Q15;
		p.anti_lm_max_order = SSLM_DAMPED_GREEDY_DEFAULT_ANTI_LM_ORDER;
		p.top_k = std::min<int32_t>(SSLM_DAMPED_GREEDY_DEFAULT_TOP_K, model->V);
		p.q_ln2 = model->dg_q_ln2;
		p.q_b = model->dg_q_b;
		p.q_c = model->dg_q_c;
	}
	*out = p;
	return SSLM_OK;
}

sslm_status sslm_stats(sslm_model model, sslm_seq seq, sslm_stats_out* out) {
	if (!model || !seq || !out) return SSLM_INVALID_ARGUMENT;
	memset(out, 0, sizeof(*out));
	// src/sslm_abi.cpp:2506-2534
	out->decode_step_ceiling = model->L;
	out->decode_step_actual = model->L;
	out->forced_token_count = seq->forced_token_count;
	out->kv_blocks_resident = 1;
	out->schema_accepting = seq->schema && schema_accepting(model->schemas[seq->schema->index], seq->walk) ? 1 : 0;
	return SSLM_OK;
}

sslm_status sslm_g5_test_only_peek_kv_block_bytes(sslm_kv_pool pool, uint32_t block_index, uint8_t* out_buf,
                                                  size_t n) {
	if (!pool || !out_buf) return SSLM_INVALID_ARGUMENT;
	if (block_index >= pool->block_count || n > pool->block_size) return SSLM_INVALID_ARGUMENT;
	return guarded([&]() -> sslm_status {
		std::lock_guard<std::mutex> lk(pool->model->mu);
		ck(hipStreamSynchronize(pool->model->tracks[0].stream));
		ck(hipMemcpy(out_buf, pool->dev + (size_t)block_index * pool->block_size, n, hipMemcpyDeviceToHost));
		return SSLM_OK;
	});
}

// Sequence blob, SSB3 (src/sslm_abi.cpp:2585-2618 layout, :2620-2720 save): 120-byte header --
// magic, model integrity hash, kv_precision, schema name hash (0: none), DFA walk state,
// adapter binding id (0), context_length, layer_index, current_token (-1 unless resting between
// decode steps), hidden scale (m, e), KV saturation count, forced-token count, anti-LM order and
// history count -- then the residual codes (H bytes, mid-token only), the anti-LM history, the
// KV block count (1) and the sequence's KV block in the reference layout.  All fields little
// endian.  The residual and KV block are read back from the device.
sslm_status sslm_seq_save(sslm_seq seq, void* buf, size_t* n) {
	if (!n || !seq) return SSLM_INVALID_ARGUMENT;
	sslm_model m = seq->model;
	const bool mid_token = seq->layer_index != 0;
	const size_t residual = mid_token ? (size_t)m->H : 0;
	const size_t history = seq->anti_lm.history.size();
	if (seq->context_length < 0 || history > (size_t)seq->context_length) return SSLM_INVALID_ARGUMENT;
	const size_t required = kBlobHeader + residual + 4 * history + 4 + seq->pool->block_size;
	if (!buf || *n < required) {
		*n = required;
		return SSLM_BUFFER_TOO_SMALL;
	}
	return guarded([&]() -> sslm_status {
		std::lock_guard<std::mutex> lk(m->mu);
		for (auto& t : m->tracks) ck(hipStreamSynchronize(t.stream));
		uint8_t* p = (uint8_t*)buf;
		Scale hs{};
		unsigned long long sat = 0;
		ck(hipMemcpy(&hs, m->stream_scale + seq->slot, sizeof(Scale), hipMemcpyDeviceToHost));
		ck(hipMemcpy(&sat, m->sat + seq->slot, 8, hipMemcpyDeviceToHost));
		memcpy(p, kBlobMagic, 4);
		memcpy(p + 4, m->art.hash, 32);
		put32(p + 36, m->c.kv_precision);
		put64(p + 40, seq->schema ? m->schemas[seq->schema->index].name_hash : 0);  // 0: no schema bound
		put32(p + 48, seq->walk);                                                     // DFA walk state
		put64(p + 52, 0);             // adapter binding id (the reference always writes 0)
		put64(p + 60, (uint64_t)seq->context_length);
		put32(p + 68, seq->layer_index);
		const bool pending_embed = seq->layer_index == 0 && !seq->ready_for_logits;
		put32(p + 72, (uint32_t)(pending_embed ? seq->current_token : -1));
		put64(p + 76, (uint64_t)hs.m);
		put64(p + 84, (uint64_t)hs.e);
		put64(p + 92, (uint64_t)sat);
		put64(p + 100, (uint64_t)seq->forced_token_count);
		put32(p + 108, (uint32_t)seq->anti_lm.order);
		put64(p + 112, (uint64_t)history);
		size_t off = kBlobHeader;
		if (residual) ck(hipMemcpy(p + off, m->stream_codes + (size_t)seq->slot * m->H, residual, hipMemcpyDeviceToHost));
		off += residual;
		for (size_t i = 0; i < history; ++i, off += 4) put32(p + off, (uint32_t)seq->anti_lm.history[i]);
		put32(p + off, 1);  // KV block count
		off += 4;
		ck(hipMemcpy(p + off, seq->pool->dev + (size_t)seq->block * seq->pool->block_size, seq->pool->block_size,
		             hipMemcpyDeviceToHost));
		off += seq->pool->block_size;
		*n = off;
		return SSLM_OK;
	});
}

// src/sslm_abi.cpp:2990-3085 with PopulateAdapterFromView (adapter_marshal.h): the adapter is an
// .sslm container (Config and SigmoidLut copied from the base, like every artifact) whose
// Provenance section starts with the 68-byte ADP1 record (magic, version 1,
// rank, target-module mask, base integrity hash, lora_alpha, use_rslora, reserved 0, name
// length), whose DeltaFoldScales entries "layer<N>.<proj>" name the adapted projections, each with
// a UFoldScales entry of `rank` rows and "<name>.lora_A" [rank, in] / "<name>.lora_B" [out, rank]
// int8 tensors.  Checks run in the reference's order; a base-hash mismatch is
// SSLM_ADAPTER_MODEL_MISMATCH, every other rejection SSLM_ARTIFACT_REJECTED.  Ranks above
// kMaxRank (64) are outside this backend's kernels and rejected as well.
sslm_status sslm_adapter_map(const void* data, size_t size, sslm_model base, sslm_adapter* out) {
	if (!out) return SSLM_INVALID_ARGUMENT;
	*out = nullptr;
	if (!data || !base) return SSLM_INVALID_ARGUMENT;
	Artifact A;
	std::string err;
	if (!parse_artifact((const uint8_t*)data, size, &A, &err)) return SSLM_ARTIFACT_REJECTED;
	const uint8_t* pv = A.provenance;
	if (!pv || A.provenance_bytes < 68 || memcmp(pv, "ADP1", 4) != 0 || rd_i32(pv + 4) != 1) return SSLM_ARTIFACT_REJECTED;
	const uint32_t rank = (uint32_t)rd_i32(pv + 8), mask = (uint32_t)rd_i32(pv + 12);
	if (rd_i32(pv + 60) != 0) return SSLM_ARTIFACT_REJECTED;
	const uint32_t name_len = (uint32_t)rd_i32(pv + 64);
	if (A.provenance_bytes < 68ull + name_len) return SSLM_ARTIFACT_REJECTED;
	if (mask & ~0x7fu) return SSLM_ARTIFACT_REJECTED;  // 7 PEFT-adaptable projections (model.h:433)
	if (memcmp(pv + 16, base->art.hash, 32) != 0) return SSLM_ADAPTER_MODEL_MISMATCH;
	if (A.weights.empty() || A.delta_fold.empty() || A.u_fold.empty()) return SSLM_ARTIFACT_REJECTED;
	if (rank > (uint32_t)kMaxRank) return SSLM_ARTIFACT_REJECTED;
	// ADP1 mask bit order: q o gate up down k v; handle slots: q k v o gate up down
	static const char* const kProj[7] = {"q_proj", "o_proj", "gate_proj", "up_proj", "down_proj", "k_proj", "v_proj"};
	static const int kSlot[7] = {0, 3, 4, 5, 6, 1, 2};
	const uint64_t H = base->H, I = base->I, KVH = base->KVH;
	const uint64_t out_ch[7] = {H, H, I, I, H, KVH, KVH};
	const uint64_t in_ch[7] = {H, H, H, H, I, H, H};
	struct Item {
		int layer, proj;
		const TensorView *a, *b, *d, *u;
	};
	std::vector<Item> items;
	for (const auto& kv : A.delta_fold) {
		const std::string& name = kv.first;
		// "layer<N>.<proj>" (adapter_marshal.h ParseLayerProjName)
		if (name.size() <= 5 || name.compare(0, 5, "layer") != 0) return SSLM_ARTIFACT_REJECTED;
		size_t i = 5;
		uint64_t layer = 0;
		while (i < name.size() && name[i] >= '0' && name[i] <= '9') {
			layer = layer * 10 + (uint64_t)(name[i] - '0');
			if (layer > 0xffffffffull) return SSLM_ARTIFACT_REJECTED;
			++i;
		}
		if (i == 5 || i >= name.size() || name[i] != '.') return SSLM_ARTIFACT_REJECTED;
		const std::string proj = name.substr(i + 1);
		if (proj.empty() || proj.find('.') != std::string::npos) return SSLM_ARTIFACT_REJECTED;
		if (layer >= (uint64_t)base->L) return SSLM_ARTIFACT_REJECTED;
		int pi = -1;
		for (int k = 0; k < 7; ++k)
			if (proj == kProj[k]) pi = k;
		if (pi < 0 || !(mask >> pi & 1)) return SSLM_ARTIFACT_REJECTED;
		if (kv.second.elems / 3 != out_ch[pi]) return SSLM_ARTIFACT_REJECTED;
		auto u = A.u_fold.find(name);
		if (u == A.u_fold.end() || u->second.elems / 3 != rank) return SSLM_ARTIFACT_REJECTED;
		auto a = A.weights.find(name + ".lora_A"), b = A.weights.find(name + ".lora_B");
		if (a == A.weights.end() || b == A.weights.end()) return SSLM_ARTIFACT_REJECTED;
		if (a->second.rank != 2 || a->second.shape[0] != rank || a->second.shape[1] != in_ch[pi]) return SSLM_ARTIFACT_REJECTED;
		if (b->second.rank != 2 || b->second.shape[0] != out_ch[pi] || b->second.shape[1] != rank) return SSLM_ARTIFACT_REJECTED;
		items.push_back(Item{(int)layer, kSlot[pi], &a->second, &b->second, &kv.second, &u->second});
	}
	auto* h = new (std::nothrow) sslm_adapter_s();
	if (!h) return SSLM_ALLOCATION_FAILED;
	const sslm_status st = guarded([&]() -> sslm_status {
		h->model = base;
		h->rank = rank;
		h->bytes = size;
		h->proj.assign((size_t)base->L * 7, AdapterProj{});
		for (const Item& it : items) {
			AdapterProj& p = h->proj[(size_t)it.layer * 7 + it.proj];
			std::vector<int8_t> a8, b8;
			std::vector<int32_t> uf, df;
			append_le(&a8, *it.a);
			append_le(&b8, *it.b);
			append_le(&uf, *it.u);
			append_le(&df, *it.d);
			p.a = dupload(a8, &h->owned);
			p.b = dupload(b8, &h->owned);
			p.ufold = dupload(uf, &h->owned);
			p.dfold = dupload(df, &h->owned);
		}
		return SSLM_OK;
	});
	if (st != SSLM_OK) {
		for (void* q : h->owned) (void)hipFree(q);
		delete h;
		return st;
	}
	base->live_refs++;
	*out = h;
	return SSLM_OK;
}

sslm_status sslm_adapter_release(sslm_adapter adapter) {
	if (!adapter) return SSLM_INVALID_ARGUMENT;
	if (adapter->live_refs.load() != 0) return SSLM_ADAPTER_HAS_LIVE_SEQUENCES;
	{
		// no decode may still read the adapter's tensors
		std::lock_guard<std::mutex> lk(adapter->model->mu);
		try {
			drop_graphs(adapter->model);  // captured graphs may hold its device pointers
		} catch (const HipError&) {
			return SSLM_INVALID_ARGUMENT;
		}
	}
	for (void* q : adapter->owned) (void)hipFree(q);
	adapter->model->live_refs--;
	delete adapter;
	return SSLM_OK;
}

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
// src/sslm_abi.cpp:2722-2987: checks in the reference's order (magic SSB3 or SSB2, sizes, model
// hash, kv precision, schema binding -- none can resolve here, as no schema is ever bound --
// field domains, exact size, KV block count, pool identity), then a block is drawn, the KV
// block and residual uploaded and the resting state rebuilt: current_token >= 0 resumes with
// the embed of that token; otherwise a whole-token state with context ready for logits (its
// residual codes are not in the blob, so they restart from zero, as in the reference).
sslm_status sslm_seq_restore(sslm_model model, sslm_kv_pool* pool, const void* buf, size_t n, sslm_seq* out) {
	if (!out) return SSLM_INVALID_ARGUMENT;
	*out = nullptr;
	if (!model || !pool || !*pool || !buf) return SSLM_INVALID_ARGUMENT;
	if (n < 4) return SSLM_INVALID_ARGUMENT;
	const uint8_t* p = (const uint8_t*)buf;
	const bool v3 = memcmp(p, kBlobMagic, 4) == 0, v2 = memcmp(p, kBlobMagicV2, 4) == 0;
	if (!v3 && !v2) return SSLM_INVALID_ARGUMENT;
	const size_t header = v3 ? kBlobHeader : kBlobHeaderV2;
	if (n < header + 4) return SSLM_INVALID_ARGUMENT;
	if (memcmp(p + 4, model->art.hash, 32) != 0) return SSLM_RESTORE_MODEL_MISMATCH;
	if (get32(p + 36) != model->c.kv_precision) return SSLM_RESTORE_KV_MISMATCH;
	// the schema binding resolves by name hash against this model's schemas, its walk state
	// inside the schema (src/sslm_abi.cpp:2755-2800)
	const uint64_t schema_hash = get64(p + 40);
	const uint32_t walk = get32(p + 48);
	sslm_schema schema = nullptr;
	if (schema_hash != 0) {
		for (size_t i = 0; i < model->schemas.size() && !schema; ++i)
			if (model->schemas[i].name_hash == schema_hash) schema = &model->schema_handles[i];
		if (!schema || walk >= model->schemas[schema->index].states) return SSLM_RESTORE_SCHEMA_MISMATCH;
	} else if (walk != kWalkUnused) {
		return SSLM_RESTORE_SCHEMA_MISMATCH;
	}
	const int64_t context_length = (int64_t)get64(p + 60);
	const uint32_t layer_index = get32(p + 68);
	const int32_t current_token = (int32_t)get32(p + 72);
	const Scale hs{(int64_t)get64(p + 76), (int64_t)get64(p + 84)};
	const uint64_t sat = get64(p + 92);
	const int64_t forced = (int64_t)get64(p + 100);
	const int32_t order = v3 ? (int32_t)get32(p + 108) : 0;
	const uint64_t history = v3 ? get64(p + 112) : 0;
	if ((order == 0 && history != 0) || order < 0 || history > (uint64_t)SIZE_MAX) return SSLM_INVALID_ARGUMENT;
	if (context_length < 0 || context_length > (int64_t)model->c.context_cap || layer_index > (uint32_t)model->L ||
	    history > (uint64_t)context_length || history > (uint64_t)model->c.context_cap)
		return SSLM_INVALID_ARGUMENT;
	const size_t residual = layer_index != 0 ? (size_t)model->H : 0;
	const size_t tail = header + residual + 4 * (size_t)history + 4;
	if (n < tail) return SSLM_INVALID_ARGUMENT;
	const uint8_t* residual_ptr = p + header;
	const uint8_t* history_ptr = residual_ptr + residual;
	if (get32(history_ptr + 4 * history) != 1) return SSLM_INVALID_ARGUMENT;  // KV block count
	const size_t block_size = model->block_bytes;
	if (block_size == 0) return SSLM_ARTIFACT_REJECTED;
	if (n < tail + block_size) return SSLM_INVALID_ARGUMENT;
	const uint8_t* kv_ptr = p + tail;
	sslm_kv_pool pl = *pool;
	if (pl->model != model) return SSLM_INVALID_ARGUMENT;
	return guarded([&]() -> sslm_status {
		std::lock_guard<std::mutex> lk(model->mu);
		uint32_t block;
		{
			std::lock_guard<std::mutex> g(pl->mu);
			if (pl->free_list.empty()) return SSLM_KV_POOL_EXHAUSTED;
			if (model->free_slots.empty()) return SSLM_ALLOCATION_FAILED;
			block = pl->free_list.back();  // src/sslm_abi.cpp:1308-1331
			pl->free_list.pop_back();
			pl->live_refs++;
		}
		const int slot = model->free_slots.back();
		model->free_slots.pop_back();
		hipStream_t st = model->tracks[0].stream;
		ck(hipStreamSynchronize(st));
		ck(hipMemcpy(pl->dev + (size_t)block * pl->block_size, kv_ptr, block_size, hipMemcpyHostToDevice));
		std::vector<int8_t> codes(model->H, 0);
		if (residual) memcpy(codes.data(), residual_ptr, residual);
		ck(hipMemcpy(model->stream_codes + (size_t)slot * model->H, codes.data(), model->H, hipMemcpyHostToDevice));
		ck(hipMemcpy(model->stream_scale + slot, &hs, sizeof(Scale), hipMemcpyHostToDevice));
		const unsigned long long sat_v = sat;
		ck(hipMemcpy(model->sat + slot, &sat_v, 8, hipMemcpyHostToDevice));
		const int32_t zero = 0;
		ck(hipMemcpy(model->status + slot, &zero, 4, hipMemcpyHostToDevice));
		sslm_seq_s* s = new sslm_seq_s();
		s->model = model;
		s->pool = pl;
		s->block = block;
		s->slot = slot;
		s->layer_index = layer_index;
		s->context_length = context_length;
		s->forced_token_count = forced;
		s->schema = schema;
		s->walk = walk;
		if (order > 0) {  // the counts are rebuilt by replaying the history (src/sslm_abi.cpp:2905-2925)
			s->anti_lm.reset(order);
			for (uint64_t i = 0; i < history; ++i) s->anti_lm.update((int32_t)get32(history_ptr + 4 * i));
		}
		if (current_token >= 0) {
			s->current_token = current_token;
			s->ready_for_logits = false;
		} else {
			s->current_token = -1;
			s->ready_for_logits = layer_index == 0 && context_length > 0;
		}
		model->live_refs++;
		{
			std::lock_guard<std::mutex> rl(g_registry_mu);
			g_live_seqs.insert(s);
		}
		*out = s;
		return SSLM_OK;
	});
}
sslm_status sslm_tokenize(sslm_model, const char*, int32_t*, int32_t*) { return SSLM_INVALID_ARGUMENT; }
// src/sslm_abi.cpp:1236-1264
sslm_status sslm_schema_lookup(sslm_model model, const char* name, sslm_schema* out) {
	if (!out) return SSLM_INVALID_ARGUMENT;
	*out = nullptr;
	if (!model || !name) return SSLM_INVALID_ARGUMENT;
	for (size_t i = 0; i < model->schemas.size(); ++i)
		if (model->schemas[i].name == name) {
			*out = &model->schema_handles[i];
			return SSLM_OK;
		}
	return SSLM_SCHEMA_NOT_FOUND;
}
size_t sslm_schema_count(sslm_model model) { return model ? model->schemas.size() : 0; }
sslm_status sslm_schema_name(sslm_model model, int32_t index, char* buf, size_t* n) {
	if (!n) return SSLM_INVALID_ARGUMENT;
	if (!model || index < 0 || (size_t)index >= model->schemas.size()) return SSLM_INVALID_ARGUMENT;
	const std::string& nm = model->schemas[index].name;
	if (!buf || *n < nm.size()) {
		*n = nm.size();
		return SSLM_BUFFER_TOO_SMALL;
	}
	memcpy(buf, nm.data(), nm.size());
	*n = nm.size();
	return SSLM_OK;
}
// src/sslm_abi.cpp:1791-1818: only a sequence that has taken no token yet, at its walk's start
sslm_status sslm_seq_set_schema(sslm_seq seq, sslm_schema schema) {
	if (!seq) return SSLM_INVALID_ARGUMENT;
	if (seq->current_token != -1) return SSLM_SCHEMA_BIND_REJECTED;
	if (seq->walk != kWalkUnused && seq->walk != 0) return SSLM_SCHEMA_BIND_REJECTED;
	if (schema && schema->model != seq->model) return SSLM_INVALID_ARGUMENT;
	seq->schema = schema;
	seq->walk = schema ? 0u : kWalkUnused;
	return SSLM_OK;
}
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
	if (!a || !w || !fold || !out_codes || !out_me || !out_status || m < 1 || m > kMaxTokens || n < 1 || k < 16 ||
	    k % 16 || n % 16 || n > kFunnelMaxN)
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
	if (!a || !w || !out || m < 1 || m > kMaxTokens || n < 1 || k < 16 || k % 16) return SSLM_INVALID_ARGUMENT;
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


// read_only: each launch is a plain streaming read of the GEMV's weight buffer (the packed copy
// where there is one) instead of the GEMV; bytes then count the weight bytes read.
static int32_t bench_gemv_pass(sslm_model model, int32_t M, int32_t iters, double* us, int64_t* bytes,
                               int64_t* shapes, int32_t cap, bool read_only) {
	if (!model || M < 1 || M > 64 || iters < 1 || cap < 1) return -1;
	sslm_model m = model;
	std::lock_guard<std::mutex> lk(m->mu);
	const sslm_status st = guarded([&]() -> sslm_status {
		Track& w = m->tracks[0];
		std::vector<TokenInfo> ti(M);
		for (int t = 0; t < M; ++t) ti[t] = TokenInfo{0, t, 0};
		ck(hipMemcpyAsync(w.tok, ti.data(), M * sizeof(TokenInfo), hipMemcpyHostToDevice, w.stream));
		ck(hipMemcpyAsync(w.lg_tok, ti.data(), M * sizeof(TokenInfo), hipMemcpyHostToDevice, w.stream));
		// every layer's four projections in the layer loop's order, then the LM head: the weights
		// stream from HBM as in a step (one layer's 46.8 MB at the 1.5B shape, 1.3 GB per pass)
		std::vector<GemmArgs> gs;
		for (int l = 0; l < m->L; ++l) {
			gs.push_back(qkv_args(m, w, l, M, nullptr, fused_attention_enabled()).g);
			gs.push_back(o_args(m, w, l, M, nullptr).g);
			gs.push_back(gu_args(m, w, l, M, nullptr).g);
			gs.push_back(down_args(m, w, l, M, nullptr).g);
		}
		gs.push_back(head_args(m, w, M, w.lg_tok));
		// The timed launches run on whatever the workspaces hold: their epilogue refusals must not
		// reach the sequences' status words, so they write a private array.
		int32_t* scratch_status = nullptr;
		ck(hipMalloc(&scratch_status, (size_t)kSlotCapacity * sizeof(int32_t)));
		ck(hipMemsetAsync(scratch_status, 0, (size_t)kSlotCapacity * sizeof(int32_t), w.stream));
		// the bytes one launch counts: algorithmic GEMV traffic, or the weight bytes a read moves
		auto launch_bytes = [&](const GemmArgs& g) -> int64_t {
			if (read_only) return g.wp ? (int64_t)sslm_launch::packed_bytes(g.N, g.K) : (int64_t)g.N * g.K;
			return (int64_t)g.N * g.K + (int64_t)g.M * g.K + 12LL * g.N + (g.epi.argmax_key ? 0 : (int64_t)g.M * g.N * 4);
		};
		int64_t seq_bytes = 0;
		for (GemmArgs& g : gs) {
			g.epi.status = scratch_status;
			seq_bytes += launch_bytes(g);
		}
		auto launch = [&](const GemmArgs& g) {
			if (read_only) sslm_launch::stream_read(g.wp ? g.wp : g.w, launch_bytes(g), scratch_status, w.stream);
			else sslm_launch::gemm(g, w.stream);
		};
		hipEvent_t a, b;
		ck(hipEventCreate(&a));
		ck(hipEventCreate(&b));
		// one timed pass set over the launches whose index i satisfies keep(i)
		auto timed = [&](auto keep) {
			for (size_t i = 0; i < gs.size(); ++i)  // warm (instruction caches, TLB)
				if (keep(i)) launch(gs[i]);
			ck(hipEventRecord(a, w.stream));
			for (int it = 0; it < iters; ++it)
				for (size_t i = 0; i < gs.size(); ++i)
					if (keep(i)) launch(gs[i]);
			ck(hipEventRecord(b, w.stream));
			ck(hipEventSynchronize(b));
			float ms = 0;
			ck(hipEventElapsedTime(&ms, a, b));
			return ms * 1e3 / iters;
		};
		us[0] = timed([](size_t) { return true; });
		bytes[0] = seq_bytes;
		shapes[0] = (int64_t)gs.size();
		if (cap >= 6) {
			const size_t head = gs.size() - 1;
			for (int c = 1; c <= 5; ++c) {
				// class c: q|k|v, o, gate|up, down (launch 4 l + c - 1 of layer l), or the LM head.
				// One class's weights (70 MB for o at the 1.5B shape) would stay in the memory-side
				// cache across repeated passes, so each timed class pass follows an untimed pass of
				// every launch, which streams 1.6 GB through it.
				auto keep = [&](size_t i) { return c == 5 ? i == head : (i < head && (int)(i % 4) == c - 1); };
				double total = 0;
				for (int it = 0; it < iters; ++it) {
					for (const GemmArgs& g : gs) launch(g);
					ck(hipEventRecord(a, w.stream));
					for (size_t i = 0; i < gs.size(); ++i)
						if (keep(i)) launch(gs[i]);
					ck(hipEventRecord(b, w.stream));
					ck(hipEventSynchronize(b));
					float ms = 0;
					ck(hipEventElapsedTime(&ms, a, b));
					total += ms * 1e3;
				}
				us[c] = total / iters;
				int64_t by = 0, n = 0;
				for (size_t i = 0; i < gs.size(); ++i)
					if (keep(i)) {
						const GemmArgs& g = gs[i];
						by += launch_bytes(g);
						++n;
					}
				bytes[c] = by;
				shapes[c] = n;
			}
		}
		(void)hipEventDestroy(a);
		(void)hipEventDestroy(b);
		ck(hipStreamSynchronize(w.stream));
		ck(hipFree(scratch_status));
		return SSLM_OK;
	});
	return st == SSLM_OK ? 1 : -1;
}

int32_t sslm_hip_bench_decode_gemv(sslm_model model, int32_t M, int32_t iters, double* us, int64_t* bytes,
                                   int64_t* shapes, int32_t cap) {
	return bench_gemv_pass(model, M, iters, us, bytes, shapes, cap, false);
}

int32_t sslm_hip_bench_read_floor(sslm_model model, int32_t M, int32_t iters, double* us, int64_t* bytes,
                                  int64_t* shapes, int32_t cap) {
	return bench_gemv_pass(model, M, iters, us, bytes, shapes, cap, true);
}

int32_t sslm_hip_bench_prefill_gemm(sslm_model model, int32_t M, int32_t iters, double* us, int64_t* ops,
                                    int64_t* launches) {
	if (!model || M < 65 || M > kMaxTokens || iters < 1 || !us || !ops || !launches) return -1;
	sslm_model m = model;
	std::lock_guard<std::mutex> lk(m->mu);
	const sslm_status st = guarded([&]() -> sslm_status {
		Track& w = m->tracks[0];
		std::vector<TokenInfo> ti(M);
		for (int t = 0; t < M; ++t) ti[t] = TokenInfo{0, 0, 0};
		ck(hipMemcpyAsync(w.tok, ti.data(), M * sizeof(TokenInfo), hipMemcpyHostToDevice, w.stream));
		// the chunk's projection GEMMs in the layer loop's order, each layer's own weights, with
		// the launch shapes (split-K planes included) the layer loop uses
		std::vector<GemmArgs> gs;
		for (int l = 0; l < m->L; ++l) {
			gs.push_back(qkv_args(m, w, l, M, nullptr, false).g);
			gs.push_back(o_args(m, w, l, M, nullptr).g);
			gs.push_back(gu_args(m, w, l, M, nullptr).g);
			gs.push_back(down_args(m, w, l, M, nullptr).g);
		}
		int32_t* scratch_status = nullptr;
		ck(hipMalloc(&scratch_status, (size_t)kSlotCapacity * sizeof(int32_t)));
		ck(hipMemsetAsync(scratch_status, 0, (size_t)kSlotCapacity * sizeof(int32_t), w.stream));
		int64_t pass_ops = 0;
		for (GemmArgs& g : gs) {
			g.epi.status = scratch_status;
			pass_ops += 2LL * g.M * g.N * g.K;
		}
		hipEvent_t a, b;
		ck(hipEventCreate(&a));
		ck(hipEventCreate(&b));
		for (const GemmArgs& g : gs) sslm_launch::gemm(g, w.stream);
		ck(hipEventRecord(a, w.stream));
		for (int i = 0; i < iters; ++i)
			for (const GemmArgs& g : gs) sslm_launch::gemm(g, w.stream);
		ck(hipEventRecord(b, w.stream));
		ck(hipEventSynchronize(b));
		float ms = 0;
		ck(hipEventElapsedTime(&ms, a, b));
		us[0] = ms * 1e3 / iters;
		ops[0] = pass_ops;
		launches[0] = (int64_t)gs.size();
		(void)hipEventDestroy(a);
		(void)hipEventDestroy(b);
		ck(hipStreamSynchronize(w.stream));
		ck(hipFree(scratch_status));
		return SSLM_OK;
	});
	return st == SSLM_OK ? 1 : -1;
}

int32_t sslm_hip_debug_site(sslm_model model, int32_t site, int32_t row, int8_t* codes, int64_t* scale_me) {
	if (!model || !codes || !scale_me || row < 0) return -1;
	sslm_model m = model;
	std::lock_guard<std::mutex> lk(m->mu);
	if (m->tracks.empty() || row >= m->tracks[0].capacity) return -1;
	const Track& w = m->tracks[0];
	const int8_t* src = nullptr;
	const Scale* sc = nullptr;
	int n = m->H;
	switch (site) {
		case 0: src = w.normed; sc = w.normed_scale; break;
		case 1: src = w.ctx; sc = w.ctx_scale; break;
		case 2: src = w.attn_stream; sc = w.attn_stream_scale; break;
		case 3: src = w.mlp_normed; sc = w.mlp_scale; break;
		case 4: src = w.act; sc = w.act_scale; n = m->I; break;
		default: return -1;
	}
	const sslm_status st = guarded([&]() -> sslm_status {
		ck(hipStreamSynchronize(w.stream));
		ck(hipMemcpy(codes, src + (size_t)row * n, n, hipMemcpyDeviceToHost));
		Scale h{};
		ck(hipMemcpy(&h, sc + row, sizeof(Scale), hipMemcpyDeviceToHost));
		scale_me[0] = h.m;
		scale_me[1] = h.e;
		return SSLM_OK;
	});
	return st == SSLM_OK ? n : -1;
}

sslm_status sslm_hip_debug_capture(sslm_model model, int32_t max_tokens) {
	if (!model || max_tokens < 0 || max_tokens > kPartLd) return SSLM_INVALID_ARGUMENT;
	sslm_model m = model;
	std::lock_guard<std::mutex> lk(m->mu);
	return guarded([&]() -> sslm_status {
		for_each_track(m, [](Track& w) { ck(hipStreamSynchronize(w.stream)); });
		if (m->dbg_codes) ck(hipFree(m->dbg_codes));
		if (m->dbg_scales) ck(hipFree(m->dbg_scales));
		m->dbg_codes = nullptr;
		m->dbg_scales = nullptr;
		m->dbg_tokens = 0;
		if (max_tokens == 0) return SSLM_OK;
		drop_graphs(m);  // captured graphs would skip the capture copies
		const int ld = std::max(m->H, m->I);
		const size_t cells = (size_t)m->L * kDbgSites * max_tokens;
		ck(hipMalloc(&m->dbg_codes, cells * ld));
		ck(hipMalloc(&m->dbg_scales, cells * sizeof(Scale)));
		ck(hipMemset(m->dbg_codes, 0, cells * ld));
		ck(hipMemset(m->dbg_scales, 0, cells * sizeof(Scale)));
		m->dbg_ld = ld;
		m->dbg_tokens = max_tokens;
		return SSLM_OK;
	});
}

int32_t sslm_hip_debug_capture_read(sslm_model model, int32_t layer, int32_t site, int32_t token, int8_t* codes,
                                    int64_t* scale_me) {
	if (!model || !codes || !scale_me) return -1;
	sslm_model m = model;
	std::lock_guard<std::mutex> lk(m->mu);
	if (!m->dbg_codes || layer < 0 || layer >= m->L || site < 0 || site >= kDbgSites || token < 0 ||
	    token >= m->dbg_tokens)
		return -1;
	const int n = (site == kDbgAct || site == kDbgGate || site == kDbgUp) ? m->I : m->H;
	const sslm_launch::SiteTap tp = dbg_tap(m, layer, site);
	const sslm_status st = guarded([&]() -> sslm_status {
		for_each_track(m, [](Track& w) { ck(hipStreamSynchronize(w.stream)); });
		ck(hipMemcpy(codes, tp.codes + (size_t)token * tp.ld, n, hipMemcpyDeviceToHost));
		Scale h{};
		ck(hipMemcpy(&h, tp.scale + token, sizeof(Scale), hipMemcpyDeviceToHost));
		scale_me[0] = h.m;
		scale_me[1] = h.e;
		return SSLM_OK;
	});
	return st == SSLM_OK ? n : -1;
}

// ---- profiling ----
void sslm_hip_profile_enable(int on) { g_prof.on = on != 0; }
void sslm_hip_profile_reset(void) {
	prof_collect();
	for (int i = 0; i < SSLM_HIP_PROFILE_CLASSES; ++i) {
		g_prof.ms[i] = 0;
		g_prof.launches[i] = g_prof.bytes[i] = g_prof.ops[i] = 0;
	}
	g_prof.shapes.clear();
}
int sslm_hip_profile_shapes(int64_t* keys, double* ms, int64_t* launches, int64_t* bytes, int64_t* ops, int cap) {
	prof_collect();
	int n = 0;
	for (auto& kv : g_prof.shapes) {
		if (n < cap) {
			if (keys) keys[n] = kv.first;
			if (ms) ms[n] = kv.second.ms;
			if (launches) launches[n] = kv.second.launches;
			if (bytes) bytes[n] = kv.second.bytes;
			if (ops) ops[n] = kv.second.ops;
		}
		++n;
	}
	return n;
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
