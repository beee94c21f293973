// .sslm v2 artifact parsing for the HIP backend (format: reference docs/sslm_format.md).
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <map>
#include <string>
#include <vector>

namespace sslm {

struct TensorView {
	const uint8_t* data = nullptr;  // little-endian elements, not necessarily aligned
	uint32_t rank = 0;
	uint32_t shape[4] = {0, 0, 0, 0};
	uint64_t elems = 0;
};

struct ConstEntry {
	int64_t v[3] = {0, 0, 0};
	uint32_t words = 0;
};

struct ModelConfig {
	uint32_t hidden = 0, layers = 0, heads = 0, kv_heads = 0, head_dim = 0, inter = 0, vocab = 0;
	uint32_t context_cap = 0, tie_embeddings = 0, kv_precision = 0, kv_block_size = 0;
};

struct Artifact {
	uint32_t flags = 0;
	uint8_t hash[32] = {0};
	ModelConfig config;
	bool has_config = false;
	std::map<std::string, TensorView> weights, biases, rope, weight_scales, delta_fold, u_fold;
	std::map<std::string, ConstEntry> composition, kv_landing_scales, kv_landing_recip;
	std::vector<int32_t> sigmoid_lut;
	const uint8_t* provenance = nullptr;
	uint64_t provenance_bytes = 0;
	// SchemaMasks (SCM1) section, parsed by the runtime
	const uint8_t* schemas = nullptr;
	uint64_t schemas_bytes = 0;
	// DampedGreedyConstants section (raw bytes; read only when header flag bit 1 is set)
	const uint8_t* damped = nullptr;
	uint64_t damped_bytes = 0;
};

// Parses and validates `data` (header, section table, SHA-256 integrity, every sub-format and
// the load-time value gate).  Returns false with a diagnostic on any rejection.  Config and
// SigmoidLut are required of every artifact, adapters included (src/artifact.cpp:152-170).
bool parse_artifact(const uint8_t* data, size_t size, Artifact* out, std::string* err);

// The canonical SIL1 table: round_half_even(sigmoid(-16 + i/32) * 2^15), i in [0, 1024].
void canonical_sigmoid_lut(int32_t out[1025]);

inline int32_t rd_i32(const uint8_t* p) {
	return (int32_t)((uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24));
}
inline int64_t rd_i64(const uint8_t* p) {
	uint64_t v = 0;
	for (int i = 0; i < 8; ++i) v |= (uint64_t)p[i] << (8 * i);
	return (int64_t)v;
}

}  // namespace sslm
