// .sslm v2 loader for the HIP backend: structure, integrity and the load-time value gate.
//
// Restates the reference's trust boundary from its normative spec and loader:
//   container  docs/sslm_format.md:47-118, src/artifact.cpp:229-410
//   manifests  docs/sslm_format.md:200-290 (WGT1/BIA1/ROP1/WSC1, KVC1), :301-365 (CFG1, SIL1)
//   values     src/model.cpp:940-1180, :1255-1330 (composition, WSC1, ROP1, KV landing, geometry)
// Reject over degrade: any deviation fails the whole load with a diagnostic.
#include "artifact.h"

#include <math.h>
#include <openssl/evp.h>
#include <string.h>

#include <algorithm>

namespace sslm {
namespace {

uint32_t rd_u32(const uint8_t* p) { return (uint32_t)rd_i32(p); }
uint64_t rd_u64(const uint8_t* p) { return (uint64_t)rd_i64(p); }

enum SecType : uint32_t {
	kConfig = 0, kProvenance = 1, kWeights = 2, kBiases = 3, kRope = 4, kScales = 5, kWeightScales = 6,
	kComposition = 7, kKvLandingScales = 8, kKvLandingRecip = 9, kCalibration = 10, kGoldenHashes = 11,
	kSigmoidLut = 12, kTokenizer = 20, kChatTemplate = 21, kUnicodeTables = 22, kSchemaMasks = 30,
	kCalibrationBand = 31, kDeltaFold = 40, kUFold = 41, kDampedGreedy = 42,
};

bool known_type(uint32_t t) {
	switch (t) {
		case kConfig: case kProvenance: case kWeights: case kBiases: case kRope: case kScales:
		case kWeightScales: case kComposition: case kKvLandingScales: case kKvLandingRecip:
		case kCalibration: case kGoldenHashes: case kSigmoidLut: case kTokenizer: case kChatTemplate:
		case kUnicodeTables: case kSchemaMasks: case kCalibrationBand: case kDeltaFold: case kUFold:
		case kDampedGreedy:
			return true;
	}
	return false;
}

// src/artifact.cpp:55-90: the one dtype each section type carries
uint32_t expected_dtype(uint32_t t) {
	switch (t) {
		case kWeights: return 1;
		case kBiases: case kRope: return 3;
		case kWeightScales: case kSigmoidLut: case kDeltaFold: case kUFold: return 2;
		default: return 0;
	}
}

uint32_t dtype_size(uint32_t d) {
	switch (d) {
		case 0: case 1: case 4: return 1;
		case 2: case 5: return 4;
		case 3: case 6: return 8;
	}
	return 0;
}

bool fail(std::string* err, const std::string& msg) {
	if (err) *err = msg;
	return false;
}

// docs/sslm_format.md:200-238
bool parse_manifest(const uint8_t* base, uint64_t size, const char* magic, uint32_t elem,
                    std::map<std::string, TensorView>* out, std::string* err) {
	if (size < 16) return fail(err, std::string(magic) + ": section shorter than 16 bytes");
	if (memcmp(base, magic, 4) != 0) return fail(err, std::string(magic) + ": bad magic");
	if (rd_u32(base + 4) != 1) return fail(err, std::string(magic) + ": unsupported version");
	const uint32_t count = rd_u32(base + 8);
	const uint32_t name_len = rd_u32(base + 12);
	if (count > 65536) return fail(err, std::string(magic) + ": too many tensors");
	const uint64_t name_start = 16 + (uint64_t)count * 48;
	const uint64_t data_region = name_start + name_len;
	if (data_region > size) return fail(err, std::string(magic) + ": descriptors/names exceed the section");
	std::vector<std::pair<uint64_t, uint64_t>> ranges;
	for (uint32_t i = 0; i < count; ++i) {
		const uint8_t* d = base + 16 + (uint64_t)i * 48;
		const uint32_t no = rd_u32(d), nl = rd_u32(d + 4), rank = rd_u32(d + 8);
		const uint64_t data_off = rd_u64(d + 28), elems = rd_u64(d + 36);
		if (rd_u32(d + 44) != 0) return fail(err, std::string(magic) + ": reserved descriptor field");
		if (nl == 0 || (uint64_t)no + nl > name_len) return fail(err, std::string(magic) + ": bad name range");
		if (rank < 1 || rank > 4) return fail(err, std::string(magic) + ": bad rank");
		TensorView tv;
		tv.rank = rank;
		uint64_t prod = 1;
		for (uint32_t r = 0; r < 4; ++r) {
			const uint32_t s = rd_u32(d + 12 + 4 * r);
			tv.shape[r] = s;
			if (r < rank) {
				if (s == 0) return fail(err, std::string(magic) + ": zero extent");
				if (prod > UINT64_MAX / s) return fail(err, std::string(magic) + ": shape overflow");
				prod *= s;
			} else if (s != 0) {
				return fail(err, std::string(magic) + ": extent past rank");
			}
		}
		if (prod != elems) return fail(err, std::string(magic) + ": elem_count != product(shape)");
		if (data_off % elem != 0 || data_off < data_region) return fail(err, std::string(magic) + ": bad data offset");
		if (elems > UINT64_MAX / elem || data_off > size || elems * elem > size - data_off)
			return fail(err, std::string(magic) + ": tensor data out of bounds");
		std::string name((const char*)base + name_start + no, nl);
		if (out->count(name)) return fail(err, std::string(magic) + ": duplicate tensor " + name);
		tv.data = base + data_off;
		tv.elems = elems;
		(*out)[name] = tv;
		ranges.push_back({data_off, data_off + elems * elem});
	}
	std::sort(ranges.begin(), ranges.end());
	for (size_t i = 1; i < ranges.size(); ++i)
		if (ranges[i].first < ranges[i - 1].second) return fail(err, std::string(magic) + ": overlapping tensors");
	return true;
}

// docs/sslm_format.md:261-288
bool parse_kvc1(const uint8_t* base, uint64_t size, uint32_t words, std::map<std::string, ConstEntry>* out,
                std::string* err) {
	if (size < 24) return fail(err, "KVC1: section shorter than 24 bytes");
	if (memcmp(base, "KVC1", 4) != 0) return fail(err, "KVC1: bad magic");
	if (rd_u32(base + 4) != 1) return fail(err, "KVC1: unsupported version");
	const uint32_t count = rd_u32(base + 8), vw = rd_u32(base + 12), name_len = rd_u32(base + 16);
	if (rd_u32(base + 20) != 0) return fail(err, "KVC1: reserved field");
	if (count > 1048576) return fail(err, "KVC1: too many entries");
	if (vw != words) return fail(err, "KVC1: value_words does not match the section type");
	const uint64_t values = 24 + (uint64_t)count * 8;
	const uint64_t names = values + (uint64_t)count * vw * 8;
	if (names + name_len > size) return fail(err, "KVC1: contents exceed the section");
	for (uint32_t i = 0; i < count; ++i) {
		const uint32_t no = rd_u32(base + 24 + 8 * i), nl = rd_u32(base + 28 + 8 * i);
		if (nl == 0 || (uint64_t)no + nl > name_len) return fail(err, "KVC1: bad name range");
		std::string name((const char*)base + names + no, nl);
		if (out->count(name)) return fail(err, "KVC1: duplicate key " + name);
		ConstEntry e;
		e.words = vw;
		for (uint32_t w = 0; w < vw; ++w) e.v[w] = rd_i64(base + values + ((uint64_t)i * vw + w) * 8);
		(*out)[name] = e;
	}
	return true;
}

// docs/sslm_format.md:301-327
bool parse_cfg1(const uint8_t* p, uint64_t size, ModelConfig* c, std::string* err) {
	if (size != 84) return fail(err, "CFG1: section is not 84 bytes");
	if (memcmp(p, "CFG1", 4) != 0) return fail(err, "CFG1: bad magic");
	if (rd_u32(p + 4) != 1) return fail(err, "CFG1: unsupported version");
	c->hidden = rd_u32(p + 8);
	c->layers = rd_u32(p + 12);
	c->heads = rd_u32(p + 16);
	c->kv_heads = rd_u32(p + 20);
	c->head_dim = rd_u32(p + 24);
	c->inter = rd_u32(p + 28);
	c->vocab = rd_u32(p + 32);
	c->context_cap = rd_u32(p + 36);
	c->tie_embeddings = rd_u32(p + 40);
	c->kv_precision = rd_u32(p + 44);
	c->kv_block_size = rd_u32(p + 48);
	if (!c->hidden || !c->layers || !c->heads || !c->kv_heads || !c->head_dim || !c->inter || !c->vocab ||
	    !c->context_cap || !c->kv_block_size)
		return fail(err, "CFG1: zero dimension");
	if (c->head_dim % 2) return fail(err, "CFG1: odd head_dim");
	if (c->tie_embeddings > 1 || c->kv_precision > 1) return fail(err, "CFG1: field outside its allowed set");
	if (rd_u32(p + 64) != 0) return fail(err, "CFG1: reserved field");
	return true;
}

bool parse_sil1(const uint8_t* p, uint64_t size, std::vector<int32_t>* lut, std::string* err) {
	if (size != 16 + 1025 * 4) return fail(err, "SIL1: wrong size");
	if (memcmp(p, "SIL1", 4) != 0) return fail(err, "SIL1: bad magic");
	if (rd_u32(p + 4) != 1) return fail(err, "SIL1: unsupported version");
	if (rd_u32(p + 8) != 1025) return fail(err, "SIL1: entry_count != 1025");
	if (rd_u32(p + 12) != 0) return fail(err, "SIL1: reserved field");
	int32_t canon[1025];
	canonical_sigmoid_lut(canon);
	lut->resize(1025);
	for (int i = 0; i < 1025; ++i) {
		(*lut)[i] = rd_i32(p + 16 + 4 * i);
		if ((*lut)[i] != canon[i]) return fail(err, "SIL1: table differs from the canonical construction");
	}
	return true;
}

bool value_gate(const Artifact& a, std::string* err) {
	for (const auto& kv : a.composition) {  // src/model.cpp:940-960
		const int64_t m = kv.second.v[0], e = kv.second.v[1];
		if (m < -(((int64_t)1 << 31) - 1) || m > ((int64_t)1 << 31) - 1 || e < -80 || e > 7)
			return fail(err, "CompositionConstants " + kv.first + " outside its domain");
	}
	for (const auto& kv : a.weight_scales) {  // src/model.cpp:976-1017
		const TensorView& t = kv.second;
		if (t.elems % 3) return fail(err, "WeightScales " + kv.first + " is not a multiple of 3");
		for (uint64_t r = 0; r < t.elems / 3; ++r) {
			const int32_t id = rd_i32(t.data + r * 12), sh = rd_i32(t.data + r * 12 + 8);
			if (id < 0 || id > 1) return fail(err, "WeightScales " + kv.first + " identity not in {0,1}");
			if (sh < 0 || sh > 31) return fail(err, "WeightScales " + kv.first + " shift outside [0,31]");
		}
	}
	for (const auto& kv : a.rope) {  // src/model.cpp:1021-1036
		for (uint64_t i = 0; i < kv.second.elems; ++i) {
			const int64_t v = rd_i64(kv.second.data + 8 * i);
			if (v < -((int64_t)1 << 30) || v > ((int64_t)1 << 30)) return fail(err, "RopeTables entry outside +-2^30");
		}
	}
	for (const auto& kv : a.kv_landing_scales) {  // src/model.cpp:1125-1140
		const int64_t m = kv.second.v[0];
		if (m < ((int64_t)1 << 30) || m > ((int64_t)1 << 31) - 1) return fail(err, "KvLandingScales m outside canonical range");
	}
	for (const auto& kv : a.kv_landing_recip) {  // src/model.cpp:1153-1176
		const int64_t e = kv.second.v[1], r = kv.second.v[2];
		if (e < -60) return fail(err, "KvLandingReciprocals e below -60");
		if (r < ((int64_t)1 << 31) + 1 || r > ((int64_t)1 << 32)) return fail(err, "KvLandingReciprocals R outside (2^31, 2^32]");
	}
	// DeltaFoldScales / UFoldScales (src/model.cpp:320-345, :380-405): (identity, mult, exponent)
	// triples, identity in {0,1}, exponent in [-31, 31]
	for (const auto* fold : {&a.delta_fold, &a.u_fold}) {
		for (const auto& kv : *fold) {
			const TensorView& t = kv.second;
			if (t.elems % 3) return fail(err, "amplifying fold " + kv.first + " is not a multiple of 3");
			for (uint64_t r = 0; r < t.elems / 3; ++r) {
				const int32_t id = rd_i32(t.data + r * 12), ex = rd_i32(t.data + r * 12 + 8);
				if (id < 0 || id > 1) return fail(err, "amplifying fold " + kv.first + " identity not in {0,1}");
				if (ex < -31 || ex > 31) return fail(err, "amplifying fold " + kv.first + " exponent outside [-31,31]");
			}
		}
	}
	if (a.has_config) {  // geometry join and ROP1 shape (src/model.cpp:1260-1330)
		const ModelConfig& c = a.config;
		if (c.kv_heads > c.heads || c.heads % c.kv_heads) return fail(err, "CFG1 kv heads do not divide heads");
		if ((uint64_t)c.heads * c.head_dim != c.hidden) return fail(err, "CFG1 hidden != heads * head_dim");
		const uint64_t expect = (uint64_t)c.context_cap * (c.head_dim / 2);
		for (const char* nm : {"cos", "sin"}) {
			auto it = a.rope.find(nm);
			if (it != a.rope.end() && it->second.elems != expect) return fail(err, "RopeTables shape does not match CFG1");
		}
	}
	return true;
}

}  // namespace

void canonical_sigmoid_lut(int32_t out[1025]) {
	for (int i = 0; i < 1025; ++i) {
		const double x = -16.0 + (double)i * (32.0 / 1024.0);
		out[i] = (int32_t)nearbyint((1.0 / (1.0 + exp(-x))) * 32768.0);  // default FE_TONEAREST: half-even
	}
}

bool parse_artifact(const uint8_t* data, size_t size, Artifact* out, std::string* err) {
	*out = Artifact{};
	if (!data) return fail(err, "null data");
	if (size < 64) return fail(err, "truncated header");
	if (memcmp(data, "SSLM", 4) != 0) return fail(err, "bad magic");
	if (rd_u32(data + 4) != 2) return fail(err, "unsupported format version");
	if (rd_u32(data + 8) != 64) return fail(err, "bad header_bytes");
	const uint32_t count = rd_u32(data + 12);
	const uint32_t flags = rd_u32(data + 16);
	if (flags & ~0x3u) return fail(err, "unknown flags bit");
	if (rd_u32(data + 20) != 0) return fail(err, "reserved header field");
	if (count > 4096) return fail(err, "too many sections");
	const uint64_t table_end = 64 + (uint64_t)count * 40;
	if (table_end > size) return fail(err, "section table truncated");
	if (rd_u64(data + 24) != size) return fail(err, "file_bytes != size");
	{  // integrity: SHA-256 over the file with the hash field zeroed (docs/sslm_format.md:26-32)
		uint8_t zero[32] = {0}, digest[32];
		unsigned int dl = 0;
		EVP_MD_CTX* ctx = EVP_MD_CTX_new();
		bool ok = ctx && EVP_DigestInit_ex(ctx, EVP_sha256(), nullptr) && EVP_DigestUpdate(ctx, data, 32) &&
		          EVP_DigestUpdate(ctx, zero, 32) && EVP_DigestUpdate(ctx, data + 64, size - 64) &&
		          EVP_DigestFinal_ex(ctx, digest, &dl);
		if (ctx) EVP_MD_CTX_free(ctx);
		if (!ok || dl != 32) return fail(err, "SHA-256 unavailable");
		if (memcmp(digest, data + 32, 32) != 0) return fail(err, "integrity SHA-256 mismatch");
		memcpy(out->hash, data + 32, 32);
	}
	out->flags = flags;
	struct Placed {
		uint32_t type;
		uint64_t off, size;
	};
	std::vector<Placed> placed;
	for (uint32_t i = 0; i < count; ++i) {
		const uint8_t* row = data + 64 + (uint64_t)i * 40;
		const uint32_t type = rd_u32(row), dtype = rd_u32(row + 4), align = rd_u32(row + 32);
		const uint64_t off = rd_u64(row + 8), bs = rd_u64(row + 16), elems = rd_u64(row + 24);
		if (rd_u32(row + 36) != 0) return fail(err, "reserved section field");
		if ((align & (align - 1)) || align < 8 || align > 4096) return fail(err, "bad section alignment");
		if (off % align) return fail(err, "misaligned section");
		const uint32_t ds = dtype_size(dtype);
		if (!ds) return fail(err, "unknown dtype");
		if (elems > UINT64_MAX / ds || elems * ds != bs) return fail(err, "byte_size != elem_count * dtype size");
		if (off > UINT64_MAX - bs || off + bs > size) return fail(err, "section out of bounds");
		if (off < table_end) return fail(err, "section overlaps the header/table");
		if (!known_type(type)) return fail(err, "unknown section type");
		if (dtype != expected_dtype(type)) return fail(err, "section dtype mismatch");
		placed.push_back({type, off, bs});
	}
	for (size_t a = 0; a < placed.size(); ++a)
		for (size_t b = a + 1; b < placed.size(); ++b) {
			if (placed[a].type == placed[b].type) return fail(err, "duplicate section");
			if (placed[a].off < placed[b].off + placed[b].size && placed[b].off < placed[a].off + placed[a].size)
				return fail(err, "overlapping sections");
		}
	bool have_cfg = false, have_sil = false;
	for (const Placed& p : placed) {
		const uint8_t* b = data + p.off;
		bool ok = true;
		switch (p.type) {
			case kConfig: ok = parse_cfg1(b, p.size, &out->config, err); have_cfg = ok; out->has_config = ok; break;
			case kSigmoidLut: ok = parse_sil1(b, p.size, &out->sigmoid_lut, err); have_sil = ok; break;
			case kWeights: ok = parse_manifest(b, p.size, "WGT1", 1, &out->weights, err); break;
			case kBiases: ok = parse_manifest(b, p.size, "BIA1", 8, &out->biases, err); break;
			case kRope: ok = parse_manifest(b, p.size, "ROP1", 8, &out->rope, err); break;
			case kWeightScales: ok = parse_manifest(b, p.size, "WSC1", 4, &out->weight_scales, err); break;
			case kComposition: ok = parse_kvc1(b, p.size, 2, &out->composition, err); break;
			case kKvLandingScales: ok = parse_kvc1(b, p.size, 2, &out->kv_landing_scales, err); break;
			case kKvLandingRecip: ok = parse_kvc1(b, p.size, 3, &out->kv_landing_recip, err); break;
			case kDeltaFold: ok = parse_manifest(b, p.size, "DFS1", 4, &out->delta_fold, err); break;
			case kUFold: ok = parse_manifest(b, p.size, "UFS1", 4, &out->u_fold, err); break;
			case kProvenance:
				out->provenance = b;
				out->provenance_bytes = p.size;
				break;
			case kSchemaMasks:
				out->schemas = b;
				out->schemas_bytes = p.size;
				break;
			case kDampedGreedy:
				out->damped = b;
				out->damped_bytes = p.size;
				break;
			default: break;
		}
		if (!ok) return false;
	}
	if (!have_cfg) return fail(err, "required Config section missing");
	if (!have_sil) return fail(err, "required SigmoidLut section missing");
	return value_gate(*out, err);
}

}  // namespace sslm
