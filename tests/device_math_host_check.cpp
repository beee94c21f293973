// Host-side check of the device integer primitives (superslm_amd/csrc/int_math.h) against
// the C oracle (oracle/sslm_oracle.c): the GPU kernels' fast formulations -- double-estimate
// reciprocal and division, 64-bit-half requant and landing, double-estimate isqrt, the
// per-element softmax -- must equal the reference restatements bit for bit.  Built and run
// by tests/test_device_math_host.py; prints "ok" and exits 0 when every case agrees.
#include <math.h>
#include <stdio.h>

#include <random>
#include <vector>

#include "../oracle/sslm_oracle.h"
#include "../superslm_amd/csrc/int_math.h"

using namespace sslm;

static long g_fail = 0;
#define EXPECT(cond, ...)                          \
	do {                                           \
		if (!(cond)) {                             \
			if (g_fail < 20) {                     \
				printf("FAIL %s: ", #cond);        \
				printf(__VA_ARGS__);               \
				printf("\n");                      \
			}                                      \
			++g_fail;                              \
		}                                          \
	} while (0)

// floor(a f + 1/2) clamped to 127, exactly: f = M 2^E with a 53-bit integer M, the product in
// 128 bits (the reference for requant_code_f's rounding logic on any non-negative double f)
static int exact_half_up(uint32_t a, double f) {
	if (a == 0 || f == 0.0) return 0;
	int E;
	const double fm = frexp(f, &E);
	const uint64_t M = (uint64_t)ldexp(fm, 53);
	E -= 53;
	const unsigned __int128 p = (unsigned __int128)a * M;
	if (E >= 0) return 127;  // a f >= 2^52
	const int sh = -E;
	if (sh > 120) return 0;  // a f < 2^-30
	const unsigned __int128 mag = (2 * p + ((unsigned __int128)1 << sh)) >> (sh + 1);
	return mag > 127 ? 127 : (int)mag;
}

int main(int argc, char** argv) {
	const long N = argc > 1 ? atol(argv[1]) : 200000;
	std::mt19937_64 rng(20261201);
	auto uni = [&](int64_t lo, int64_t hi) { return lo + (int64_t)(rng() % (uint64_t)(hi - lo + 1)); };

	// reciprocal: canonical domain exhaustively at the ends, randomly inside; the rest replays Newton
	for (int64_t dn = (1LL << 30); dn < (1LL << 30) + 4096; ++dn) EXPECT(reciprocal_fast(dn) == or_reciprocal(dn), "%lld", (long long)dn);
	for (int64_t dn = (1LL << 31) - 4096; dn < (1LL << 31); ++dn) EXPECT(reciprocal_fast(dn) == or_reciprocal(dn), "%lld", (long long)dn);
	for (long i = 0; i < N; ++i) {  // callers pass canonical or int32-range mantissas (fits_i32)
		const int64_t dn = i % 10 ? uni(1LL << 30, (1LL << 31) - 1) : uni(-(1LL << 31), (1LL << 31) - 1);
		EXPECT(reciprocal_fast(dn) == or_reciprocal(dn), "%lld", (long long)dn);
	}
	// floor division by double estimate
	for (long i = 0; i < N; ++i) {
		const int bits = (int)uni(1, 62);
		const int64_t n = uni(0, (int64_t)((1ULL << bits) - 1));
		const int64_t d = i % 3 ? uni(1, 1LL << (int)uni(0, 62)) : uni(1, 300);
		EXPECT(div_floor_pos(n, d) == n / d, "%lld / %lld", (long long)n, (long long)d);
	}
	// isqrt
	for (long i = 0; i < N; ++i) {
		const int bits = (int)uni(0, 63);
		const int64_t n = bits == 63 ? uni(0, INT64_MAX) : uni(0, (int64_t)((1ULL << bits) - 1));
		EXPECT(isqrt_fast(n) == or_isqrt(n), "%lld", (long long)n);
	}
	for (int64_t r = 0; r < 100000; ++r)
		for (int64_t d = -1; d <= 1; ++d) {
			const int64_t n = r * r + d;
			if (n >= 0) EXPECT(isqrt_fast(n) == or_isqrt(n), "%lld", (long long)n);
		}
	// requant code on the funnel's domain
	for (long i = 0; i < N; ++i) {
		const int64_t x = uni(-(1LL << 31), 1LL << 31);
		const int64_t dn = uni(1LL << 30, (1LL << 31) - 1);
		const int64_t r = or_reciprocal(dn);
		const int s = (int)uni(-1, 30);
		EXPECT(requant_code_small(x, (uint64_t)r, s) == or_requant_code_wide(x, r, s), "%lld %lld %d", (long long)x,
		       (long long)r, s);
		EXPECT(requant_code_f(x, requant_factor(r, s)) == or_requant_code_wide(x, r, s), "f %lld %lld %d", (long long)x,
		       (long long)r, s);
	}
	// the double form at the rounding boundaries: x around (n - 1/2) 2^(62-s) / (127 r) for every
	// code n (a third of the cases with r near 2^32)
	for (long i = 0; i < N / 4; ++i) {
		const int64_t dn = i % 3 ? uni(1LL << 30, (1LL << 31) - 1) : (1LL << 30) + uni(0, 64);
		const int64_t r = or_reciprocal(dn);
		const int s = (int)uni(-1, 30);
		const int n = (int)uni(0, 128);
		const long double xb = ((long double)n - 0.5L) * ldexpl(1.0L, 62 - s) / (127.0L * (long double)r);
		const int64_t x0 = (int64_t)floorl(xb);
		for (int64_t d = -2; d <= 2; ++d) {
			const int64_t xa = x0 + d;
			if (xa < 0 || xa > (1LL << 31)) continue;
			for (int sg = 0; sg < 2; ++sg) {
				const int64_t x = sg ? -xa : xa;
				EXPECT(requant_code_f(x, requant_factor(r, s)) == or_requant_code_wide(x, r, s), "edge %lld %lld %d",
				       (long long)x, (long long)r, s);
			}
		}
	}
	// requant_code_f's rounding logic for any double factor, within a few ulps of every
	// half-integer m - 1/2 (where the product's rounding error decides the code)
	for (long i = 0; i < N / 2; ++i) {
		const uint32_t a = (uint32_t)(i % 4 ? uni(1, 1LL << 31) : uni(1, 4096));
		const int m = (int)uni(1, 128);
		double f = ((double)m - 0.5) / (double)a;
		for (int st = 0; st < 3; ++st) f = nextafter(f, 0.0);
		for (int st = 0; st < 7; ++st, f = nextafter(f, 1e300))
			for (int sg = 0; sg < 2; ++sg) {
				const int64_t x = sg ? -(int64_t)a : (int64_t)a;
				const int want = exact_half_up(a, f);
				EXPECT(requant_code_f(x, f) == (int8_t)(sg ? -want : want), "near tie a=%u m=%d f=%.17g", a, m, f);
			}
	}
	// exact ties: q = 127 x r / 2^(62-s) is a half-integer below 128 only at q = 63.5 (127 must
	// divide 2m - 1), i.e. x r = 2^(61-s): r = 2^32, x = 2^(29-s).  Every such input, both signs.
	for (int s = -1; s <= 29; ++s)
		for (int sg = 0; sg < 2; ++sg) {
			const int64_t r = 1LL << 32, x = (sg ? -1 : 1) * (1LL << (29 - s));
			EXPECT(requant_code_f(x, requant_factor(r, s)) == or_requant_code_wide(x, r, s), "tie %lld %d", (long long)x, s);
			EXPECT(or_requant_code_wide(x, r, s) == (sg ? -64 : 64), "tie rounds away from zero");
		}
	// landing on residual operands, every exponent band
	for (long i = 0; i < N; ++i) {
		const int64_t branch = uni(-127, 127);
		const int64_t m_a = i % 7 ? uni(-(1LL << 31), 1LL << 31) : uni(-(1LL << 40), 1LL << 40);
		const int64_t r_t = i % 5 ? uni((1LL << 31) + 1, 1LL << 32) : uni(1, 1LL << 34);
		const int64_t e_a = uni(-150, 50), e_t = uni(-150, 50);
		const int64_t k = composed_exponent(e_a, e_t);
		bool cl1, ex1;
		const int64_t v1 = landing_small(branch, m_a, r_t, k, &cl1, &ex1);
		uint64_t sat = 0;
		int ex2 = 0;
		const int64_t v2 = or_landing_rescale(branch, m_a, r_t, e_a, e_t, &sat, &ex2);
		EXPECT(v1 == v2 && (uint64_t)cl1 == sat && (int)ex1 == ex2, "%lld %lld %lld %lld %lld", (long long)branch,
		       (long long)m_a, (long long)r_t, (long long)e_a, (long long)e_t);
		bool cl3, ex3;
		const int64_t v3 = landing_rescale(branch * 1000003, m_a, r_t, k, &cl3, &ex3);
		sat = 0;
		const int64_t v4 = or_landing_rescale(branch * 1000003, m_a, r_t, e_a, e_t, &sat, &ex2);
		EXPECT(v3 == v4 && (uint64_t)cl3 == sat && (int)ex3 == ex2, "wide branch");
	}
	// funnel: scale plan + codes against RequantChainChecked
	for (long i = 0; i < N / 20; ++i) {
		const int n = (int)uni(1, 64);
		const int64_t mag = (int64_t[]){1, 127, 1LL << 20, 1LL << 31, (1LL << 31) + 1}[uni(0, 4)];
		std::vector<int64_t> row(n);
		uint64_t dmax = 0;
		for (auto& v : row) {
			v = uni(-mag, mag);
			const uint64_t a = v < 0 ? (uint64_t)0 - (uint64_t)v : (uint64_t)v;
			dmax = a > dmax ? a : dmax;
		}
		const int n_in = (int)uni(0, 2);
		Scale inc[2];
		or_scale oinc[2];
		for (int j = 0; j < n_in; ++j) {
			inc[j] = Scale{uni(1LL << 30, (1LL << 31) - 1), uni(-80, 8)};
			oinc[j] = or_scale{inc[j].m, inc[j].e};
		}
		const Scale site{i % 50 ? uni(1LL << 30, (1LL << 31) - 1) : uni(1, 1LL << 32), uni(-80, 8)};
		FunnelPlan plan;
		const int32_t st = funnel_plan(dmax, inc, n_in, site, &plan);
		std::vector<int8_t> codes(n);
		or_scale out;
		const int ost = or_requant_chain(row.data(), n, oinc, n_in, or_scale{site.m, site.e}, codes.data(), &out);
		EXPECT(st == ost, "status %d vs %d", st, ost);
		if (st == 0 && ost == 0) {
			EXPECT(plan.out.m == out.m && plan.out.e == out.e, "scale");
			for (int j = 0; j < n; ++j) EXPECT(requant_code_small(row[j], (uint64_t)plan.r, plan.s) == codes[j], "code");
			const double f = requant_factor(plan.r, plan.s);
			for (int j = 0; j < n; ++j) EXPECT(requant_code_f(row[j], f) == codes[j], "code f");
		}
	}
	// softmax row as the attention kernel computes it (constants, gate, per-element i-exp, Q15)
	int64_t ln2_q, b_q, ca_q;
	or_iexp_pinned(&ln2_q, &b_q, &ca_q);
	long rows_ok = 0;
	for (long i = 0; i < N / 50; ++i) {
		const int64_t m = uni(1LL << 30, (1LL << 31) - 1), e = uni(-75, -20);
		int64_t a1, a2, a3, b1, b2, b3;
		const int d1 = iexp_scale_constants(m, e, ln2_q, b_q, ca_q, &a1, &a2, &a3);
		const int d2 = or_iexp_scale_constants(m, e, ln2_q, 30, b_q, 30, ca_q, 30, &b1, &b2, &b3);
		EXPECT((d1 == 0) == (d2 == 0), "constants status");
		if (d1 || d2) continue;
		EXPECT(a1 == b1 && a2 == b2 && a3 == b3, "constants");
		const int width = (int)uni(1, 400);
		const int32_t gate = check_softmax_width(a2, a3, width);
		EXPECT((gate == 0) == (or_check_softmax_width(a2, a3, width) == 0), "gate");
		if (gate) continue;
		std::vector<int64_t> sc(width), po(width);
		int64_t mx = INT64_MIN;
		for (auto& v : sc) {
			v = uni(-(1LL << 21), 1LL << 21);
			mx = v > mx ? v : mx;
		}
		const int ok = or_softmax_row_q15(sc.data(), width, a1, a2, a3, po.data());
		const int64_t M = softmax_ceiling(a2, a3);
		bool refused = false;
		int64_t total = 0;
		std::vector<int64_t> ev(width);
		for (int j = 0; j < width; ++j) {
			ev[j] = iexp_element(sc[j] - mx, a1, a2, a3, M);
			if (ev[j] < 0) refused = true;
			else total += ev[j];
		}
		EXPECT(refused == !ok, "refusal");
		if (refused || !ok) continue;
		const int64_t den = total > 1 ? total : 1;
		for (int j = 0; j < width; ++j) EXPECT(div_floor_pos(ev[j] << 15, den) == po[j], "prob");
		++rows_ok;
	}
	EXPECT(rows_ok > 100, "too few accepted softmax rows: %ld", rows_ok);
	// bias term, SiLU lookup, folds, RoPE
	std::vector<int32_t> table(1025);
	for (int j = 0; j < 1025; ++j) table[j] = (int32_t)(j * 32);  // any monotone table exercises the lookup
	for (long i = 0; i < N; ++i) {
		const int64_t b = (i & 1) ? uni(-(1LL << 40), 1LL << 40) : uni(-(1LL << 30) + 1, (1LL << 30) - 1), r_a = uni((1LL << 31) + 1, 1LL << 32), e_a = uni(-120, 10);
		const int64_t acc = uni(-(1LL << 62), 1LL << 62);
		int64_t t1 = 0, t2 = 0;
		const bool k1 = bias_term(b, r_a, e_a, acc, &t1);
		const int k2 = or_bias_reconcile_wide(b, 30, r_a, e_a, &t2);
		if (k2) {
			const uint64_t s = (uint64_t)acc + (uint64_t)t2;
			const bool ovf = ((((uint64_t)acc ^ (uint64_t)t2) >> 63) == 0) && ((((uint64_t)acc ^ s) >> 63) != 0);
			EXPECT(k1 == !ovf && (!k1 || t1 == t2), "bias");
		} else {
			EXPECT(!k1, "bias domain");
		}
		const int8_t code = (int8_t)uni(-128, 127);
		const int64_t m = uni(1LL << 30, (1LL << 31) - 1);
		const int ee = (int)uni(-60, 5);
		EXPECT(silu_sigmoid_q15(table.data(), code, m, ee) == or_silu_sigmoid_q15(table.data(), code, m, ee), "silu");
		const int64_t a64 = uni(-(1LL << 40), 1LL << 40);
		const int32_t id = (int32_t)(i % 10 == 0), mult = (int32_t)uni(1LL << 30, (1LL << 31) - 1);
		const int32_t sh = (int32_t)uni(0, 31), ex = (int32_t)uni(-31, 31);
		EXPECT(apply_fold(a64, id, mult, sh) == or_apply_fold(a64, id, mult, sh), "fold");
		EXPECT(apply_amp_fold(a64, id, mult, ex) == or_apply_amp_fold(a64, id, mult, ex), "amp fold");
		// the bounded GEMM-epilogue fold: |acc| <= 2^29, any int32 multiplier, shifts 0..31
		const int32_t ab = (i % 7 == 0) ? (int32_t)((i & 8) ? (1 << 29) : -(1 << 29)) : (int32_t)uni(-(1LL << 29), 1LL << 29);
		const int32_t mb = (i % 5 == 0) ? (int32_t)((i & 16) ? INT32_MAX : INT32_MIN) : (int32_t)uni(INT32_MIN, INT32_MAX);
		const int32_t sb = (int32_t)(i % 32);
		EXPECT(fold_bounded(ab, fold_consts(id, mb, sb)) == or_apply_fold(ab, id, mb, sb), "bounded fold %d %d %d", ab, mb, sb);
		const int32_t x = (int32_t)uni(-127, 127), y = (int32_t)uni(-127, 127);
		const int32_t c = (int32_t)uni(-(1LL << 30), 1LL << 30), s = (int32_t)uni(-(1LL << 30), 1LL << 30);
		int64_t x1, y1, x2, y2;
		rope_pair(x, y, c, s, &x1, &y1);
		or_rope_pair(x, y, c, s, &x2, &y2);
		EXPECT(x1 == x2 && y1 == y2, "rope");
	}
	if (g_fail) {
		printf("%ld failures\n", g_fail);
		return 1;
	}
	printf("ok\n");
	return 0;
}
