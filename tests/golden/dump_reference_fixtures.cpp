// Emits, as JSON on stdout, the golden vectors the reference's own unit tests hold for the
// integer forward path (inputs and expected outputs only).  Built and run by
// make_fixtures.py in a container where the reference tree is present; the committed output
// (reference_fixtures.json) is what the tests read.  The fixture headers are included from
// the reference tree by path -- nothing of them is copied here.
#include <cinttypes>
#include <cstdio>
#include <string>

#include "matmul_golden_pin.h"
#include "silu_lut_golden_table.h"
#include "sslm_iexp_domain_fixtures.h"
#include "sslm_intmath_fixtures.h"
#include "sslm_matmul_fixtures.h"
#include "sslm_s3_1_c30_iexp_domain_sweep_fixtures.h"
#include "sslm_s3_1_wide_intmath_fixtures.h"
#include "sslm_s3_2_fixtures.h"
#include "sslm_s3_3_fixtures.h"
#include "sslm_s3_3_rope_application_site_fixtures.h"

using namespace superslm_test;

namespace {
bool g_first = true;
void key(const char* k) {
	std::printf("%s\"%s\":", g_first ? "" : ",", k);
	g_first = false;
}
void sep(size_t i) {
	if (i) std::printf(",");
}
void str(const char* s) { std::printf("\"%s\"", s ? s : ""); }
template <typename T>
void arr(const T* p, size_t n) {
	std::printf("[");
	for (size_t i = 0; i < n; ++i) {
		sep(i);
		std::printf("%lld", (long long)p[i]);
	}
	std::printf("]");
}
#define ROWS(name, table, count, body)              \
	key(name);                                      \
	std::printf("[");                               \
	for (size_t i = 0; i < (count); ++i) {          \
		const auto& c = (table)[i];                 \
		sep(i);                                     \
		std::printf("{");                           \
		body;                                       \
		std::printf("}");                           \
	}                                               \
	std::printf("]");
#define I(f) std::printf("\"" #f "\":%lld,", (long long)(c.f))
#define U(f) std::printf("\"" #f "\":%llu,", (unsigned long long)(c.f))
#define B(f) std::printf("\"" #f "\":%s,", (c.f) ? "true" : "false")
#define S(f) (std::printf("\"" #f "\":"), str(c.f), std::printf(","))
#define A(f, n) (std::printf("\"" #f "\":"), arr(c.f, n), std::printf(","))
#define END std::printf("\"_\":0")
}  // namespace

int main() {
	std::printf("{");
	ROWS("srdhm", kC2Cases, kC2CasesCount, (S(label), I(a), I(b), I(expected), END));
	ROWS("rdbpot", kC1C3Cases, kC1C3CasesCount, (S(label), I(x), I(exponent), I(expected), END));
	ROWS("mbqm", kMbqmCases, kMbqmCasesCount, (S(label), I(x), I(multiplier), I(shift), I(expected), END));
	ROWS("clz64", kClz64Cases, kClz64CasesCount, (S(label), U(n), I(expected), END));
	ROWS("max_abs", kMaxAbsCases, kMaxAbsCasesCount, (S(label), A(data, c.n), I(expected), END));
	ROWS("normalize_scale", kNormalizeScaleCases, kNormalizeScaleCasesCount,
	     (S(label), I(d_prime), I(expected_dn), I(expected_s), END));
	ROWS("reciprocal_named", kDynRecipNamedCases, kDynRecipNamedCasesCount, (S(label), I(dn), I(expected_r), END));
	ROWS("reciprocal_dense", kDynRecipDenseCases, kDynRecipDenseCasesCount, (I(dn), I(expected_r), END));
	ROWS("requant", kRequantCases, kRequantCasesCount, (S(label), I(x_i), I(r), I(s), I(expected), END));
	ROWS("pipeline", kPipelineCases, kPipelineCasesCount,
	     (S(label), A(xs, c.n), A(expected_codes, c.n), I(expected_d_prime), I(expected_dn), I(expected_s),
	      I(expected_r), END));
	ROWS("isqrt", kISqrtCases, kISqrtCasesCount, (S(label), I(n), I(expected_root), END));
	ROWS("shift_by_max", kShiftByMaxCases, kShiftByMaxCasesCount, (S(label), A(logits, c.n), A(expected, c.n), END));
	ROWS("iexp", kIExpCases, kIExpCasesCount, (S(label), I(q), I(q_ln2), I(q_b), I(q_c), I(expected), END));
	ROWS("rope", kRopeCases, kRopeCasesCount,
	     (S(label), I(x), I(y), I(cos_q30), I(sin_q30), I(expected_x), I(expected_y), END));
	ROWS("max_abs_wide", kMaxAbsWideCases, sizeof(kMaxAbsWideCases) / sizeof(kMaxAbsWideCases[0]),
	     (S(label), A(data, c.n), I(expected), END));
	ROWS("requant_wide", kRequantWideCases, sizeof(kRequantWideCases) / sizeof(kRequantWideCases[0]),
	     (S(label), I(x_i), I(r), I(s), I(expected), END));
	ROWS("iexp_construct", kIExpConstructCases, sizeof(kIExpConstructCases) / sizeof(kIExpConstructCases[0]),
	     (S(label), I(q), I(q_ln2), I(q_b), I(q_c), S(expected_domain), I(expected_z), I(expected_base),
	      I(expected_value), END));
	ROWS("iexp_domain", kIExpDomainCases, sizeof(kIExpDomainCases) / sizeof(kIExpDomainCases[0]),
	     (S(label), I(q), I(q_ln2), I(q_b), I(q_c), B(expected_in_domain), END));
	ROWS("iexp_scale_sweep", kC30IExpDomainSweepCases,
	     sizeof(kC30IExpDomainSweepCases) / sizeof(kC30IExpDomainSweepCases[0]),
	     (I(m), I(e), B(derivation_ok), I(q_ln2), I(q_b), I(q_c), B(expected_in_domain), END));
	ROWS("softmax_width", kC32WidthDomainCases, kC32WidthDomainCasesCount,
	     (S(label), I(m), I(e), I(q_ln2), I(q_b), I(q_c), I(row_max), I(width), B(shipped_check_ok),
	      B(ok_under_2pow47), END));
	{
		const C32WidthDomainCase* band = &kC32BandCase;
		ROWS("softmax_width_band", band, 1,
		     (S(label), I(q_b), I(q_c), I(row_max), I(width), B(ok_under_2pow47), END));
	}
	ROWS("landing", kLandingCompositeCases, kLandingCompositeCasesCount,
	     (S(label), I(branch_code), I(m_b), I(r_h), I(e_b), I(e_h), I(correct_raw), I(correct), END));
	{
		const RopeSitePositionCase* cases[2] = {&kRopeSitePositionZeroCase, &kRopeSitePositionCapMinusOneCase};
		ROWS("rope_site", cases, 2,
		     (std::printf("\"label\":"), str(c->label), std::printf(","), std::printf("\"position\":%lld,", (long long)c->position),
		      std::printf("\"row\":"), arr(c->row, 128), std::printf(",\"cos_row\":"), arr(c->cos_row, 64),
		      std::printf(",\"sin_row\":"), arr(c->sin_row, 64), std::printf(",\"expected_out\":"),
		      arr(c->expected_out, 128), std::printf(","), END));
	}
	ROWS("floor_div", kC31UnitCases, kC31UnitCasesCount, (I(hidden), I(roots), I(floor_q), I(trunc_q), END));
	ROWS("matmul_rows", kRowCases, kRowCasesCount,
	     (S(label), I(in_channels), I(out_channels), A(activations, c.in_channels),
	      A(weights, c.in_channels * c.out_channels), A(expected, c.out_channels), END));
	ROWS("matmul_tail", kTailSweepCases, sizeof(kTailSweepCases) / sizeof(kTailSweepCases[0]),
	     (S(label), I(in_channels), I(out_channels), A(activations, c.in_channels),
	      A(weights, c.in_channels * c.out_channels), A(expected, c.out_channels), END));
	ROWS("matmul_multirow", kMultiRowCases, sizeof(kMultiRowCases) / sizeof(kMultiRowCases[0]),
	     (S(label), I(num_tokens), I(in_channels), I(out_channels), A(activations, c.num_tokens * c.in_channels),
	      A(weights, c.in_channels * c.out_channels), A(expected, c.num_tokens * c.out_channels), END));
	ROWS("matmul_composition", kCompositionCases, sizeof(kCompositionCases) / sizeof(kCompositionCases[0]),
	     (S(label), I(in_channels), I(out_channels), A(activations, c.in_channels),
	      A(weights, c.in_channels * c.out_channels), A(golden_i32, c.out_channels), I(expected_d_prime),
	      I(expected_dn), I(expected_s), I(expected_r), A(expected_codes, c.out_channels), END));
	ROWS("matmul_uniform", kUniformCases, sizeof(kUniformCases) / sizeof(kUniformCases[0]),
	     (S(label), I(in_channels), I(act_value), I(wgt_value), I(expected), END));
	ROWS("matmul_golden", kMatmulGoldenCases, sizeof(kMatmulGoldenCases) / sizeof(kMatmulGoldenCases[0]),
	     (S(label), U(seed), I(in_channels), I(out_channels), I(num_tokens), I(kind), B(int32_safe), END));
	key("matmul_golden_lcg_probe");
	arr(kMatmulGoldenLcgProbe, 16);
	key("matmul_golden_total_bytes");
	std::printf("%zu", kMatmulGoldenTotalBytes);
	key("matmul_golden_sha256");
	str(kMatmulGoldenHash);
	key("silu_table");
	arr(kSiluLutGoldenTable, 1025);
	std::printf("}\n");
	return 0;
}
