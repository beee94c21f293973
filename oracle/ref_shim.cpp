// C-linkage doors onto the compiled reference's per-primitive C++ functions -- TEST
// INFRASTRUCTURE ONLY.  Built by oracle/Makefile together with the reference's own sources
// (read in place under /root/reference, never copied) into oracle/_ref/libsuperslm_ref.so, so
// the CPU tests can compare the C restatement in sslm_oracle.c against the reference primitive
// by primitive on random inputs.  The reference's own sslm_* C ABI is exported by the same .so.
#include <cpuid.h>

#include <cstdint>
#include <span>

#include "superslm/checked_chain_funnel.h"
#include "superslm/forward_sites.h"
#include "superslm/intmath.h"
#include "superslm/matmul.h"
#include "superslm/silu_lut.h"
#include "superslm/silu_lut_canonical.h"

using superslm::CarriedScale;

extern "C" {

int ref_requant_chain(const int64_t* row, size_t n, const int64_t* in_me, size_t n_in, int64_t site_m,
                      int64_t site_e, int8_t* out_codes, int64_t* out_me) {
	CarriedScale inc[8];
	for (size_t i = 0; i < n_in && i < 8; ++i) inc[i] = CarriedScale{in_me[2 * i], in_me[2 * i + 1]};
	CarriedScale out{};
	auto r = superslm::RequantChainChecked(row, n, std::span<const CarriedScale>(inc, n_in),
	                                       CarriedScale{site_m, site_e}, out_codes, &out);
	out_me[0] = out.m;
	out_me[1] = out.e;
	return static_cast<int>(r.status);
}

int64_t ref_reciprocal(int64_t dn) { return superslm::CarriedScaleReciprocal(dn); }

int ref_iexp_scale_constants(int64_t m, int64_t e, int64_t* out3) {
	return static_cast<int>(superslm::IExpScaleConstants(m, e, superslm::kIExpLn2Q, 30, superslm::kIExpBQ, 30,
	                                                     superslm::kIExpCaQ, 30, &out3[0], &out3[1],
	                                                     &out3[2]));
}

int ref_softmax_row(const int64_t* scores, size_t width, int64_t q_ln2, int64_t q_b, int64_t q_c,
                    int64_t* out) {
	return superslm::SoftmaxRowQ15(scores, width, q_ln2, q_b, q_c, out) ? 1 : 0;
}

int ref_check_softmax_width(int64_t q_b, int64_t q_c, size_t width) {
	return static_cast<int>(superslm::CheckSoftmaxRowWidthDomain(q_b, q_c, width));
}

int64_t ref_landing_rescale(int64_t branch, int64_t m_a, int64_t r_t, int64_t e_a, int64_t e_t,
                            uint64_t* sat, int* exceeded) {
	bool ex = false;
	int64_t v = superslm::LandingRescale(branch, m_a, r_t, e_a, e_t, sat, &ex);
	*exceeded = ex ? 1 : 0;
	return v;
}

int ref_rmsnorm(const int8_t* h, const int32_t* g, size_t n, int64_t site_m, int64_t site_e, int8_t* out,
                int64_t* out_me) {
	CarriedScale o{};
	auto st = superslm::RmsNormSite(h, g, n, CarriedScale{}, CarriedScale{site_m, site_e}, out, &o);
	out_me[0] = o.m;
	out_me[1] = o.e;
	return static_cast<int>(st);
}

int ref_mlp_act(const int8_t* gate, int64_t gm, int64_t ge, const int8_t* up, int64_t um, int64_t ue, size_t n,
                int64_t site_m, int64_t site_e, int8_t* out, int64_t* out_me) {
	CarriedScale o{};
	auto st = superslm::MlpActSite(gate, CarriedScale{gm, ge}, up, CarriedScale{um, ue}, n,
	                               superslm::kSiluLutCanonicalTable, CarriedScale{site_m, site_e}, out, &o);
	out_me[0] = o.m;
	out_me[1] = o.e;
	return static_cast<int>(st);
}

int ref_residual(const int8_t* branch, int64_t bm, int64_t be, const int8_t* stream, int64_t sm, int64_t se,
                 size_t n, int64_t site_m, int64_t site_e, int8_t* out, int64_t* out_me) {
	CarriedScale o{};
	auto st = superslm::ResidualReconcileSite(branch, CarriedScale{bm, be}, stream, CarriedScale{sm, se}, n,
	                                          CarriedScale{site_m, site_e}, out, &o);
	out_me[0] = o.m;
	out_me[1] = o.e;
	return static_cast<int>(st);
}

int32_t ref_silu_sigmoid(int8_t code, int64_t m, int e) {
	return superslm::SiluSigmoidQ15(superslm::kSiluLutCanonicalTable, code, m, e);
}

const int32_t* ref_silu_table(void) { return superslm::kSiluLutCanonicalTable; }

int64_t ref_apply_fold(int64_t acc, int32_t id, int32_t mult, int32_t shift) {
	return superslm::ApplyWeightScaleFold(acc, id, mult, shift);
}

int64_t ref_apply_amp_fold(int64_t acc, int32_t id, int32_t mult, int32_t exponent) {
	return superslm::ApplyAmplifyingWeightScaleFold(acc, id, mult, exponent);
}

int ref_bias_reconcile_wide(int64_t b, int64_t q_b, int64_t r_a, int64_t e_a, int64_t* out) {
	return superslm::BiasReconcileWide(b, q_b, r_a, e_a, out) ? 1 : 0;
}

void ref_rope_pair(int32_t x, int32_t y, int32_t c, int32_t s, int64_t* out2) {
	auto p = superslm::RopeApplyPair(x, y, c, s);
	out2[0] = p.x;
	out2[1] = p.y;
}

void ref_gemm_i8(const int8_t* a, const int8_t* w, size_t m, size_t k, size_t n, int64_t* out) {
	superslm::GemmInt8Accumulate(a, w, m, k, n, out);
}

// The matmul tier the reference's dispatch selects on this host: this host's CPUID / XGETBV
// fields through the reference's own resolver (0 SSE2, 1 AVX2, 2 AVX-512).
int ref_dot_row_tier(void) {
	unsigned a = 0, b = 0, c = 0, d = 0;
	__get_cpuid_count(0, 0, &a, &b, &c, &d);
	const int max_leaf = (int)a;
	unsigned c1 = 0;
	__get_cpuid_count(1, 0, &a, &b, &c1, &d);
	unsigned b7 = 0;
	if (max_leaf >= 7) __get_cpuid_count(7, 0, &a, &b7, &c, &d);
	unsigned long long xcr0 = 0;
	if (c1 & (1u << 27)) {
		unsigned lo = 0, hi = 0;
		__asm__ volatile("xgetbv" : "=a"(lo), "=d"(hi) : "c"(0));
		xcr0 = ((unsigned long long)hi << 32) | lo;
	}
	return superslm::ResolveDotRowTier(max_leaf, (int)c1, (int)b7, xcr0);
}

}  // extern "C"
