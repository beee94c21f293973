// Integer primitives of SuperSLM's forward path, shared by host and device code.
//
// Each function restates the reference primitive cited beside it (paths relative to the
// reference root) and must stay bit-identical to it: the GPU results are compared byte for byte
// against the CPU path.  128-bit intermediates use clang's __int128, which the AMDGPU backend
// lowers to 64-bit pairs.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#define SSLM_HD __host__ __device__ __forceinline__
// Rarely taken slow paths stay out of line: a kernel's latency-bound row code runs once per
// launch from a cold instruction cache, so its size costs more than a call on the rare path.
#define SSLM_COLD __host__ __device__ inline __attribute__((noinline))

namespace sslm {

typedef __int128 s128;
typedef unsigned __int128 u128;

constexpr int32_t kI32Min = -2147483647 - 1;
constexpr int32_t kI32Max = 2147483647;
constexpr int64_t kI64Max = 0x7fffffffffffffffLL;
constexpr int64_t kI64Min = -kI64Max - 1;
constexpr int64_t kSoftmaxMaxSafe = ((int64_t)1 << 62) >> 15;  // checked_chain_funnel.h:563

struct Scale {
	int64_t m;
	int64_t e;
};

// src/intmath.cpp:230-236
SSLM_HD int32_t srdhm(int32_t a, int32_t b) {
	int64_t ab = (int64_t)a * (int64_t)b;
	int64_t r = (ab + ((int64_t)1 << 30)) >> 31;
	return r > kI32Max ? kI32Max : (int32_t)r;
}

// src/intmath.cpp:244-251 (int32 instance): x / 2^e, ties away from zero, e in [0,31]
SSLM_HD int32_t rdbpot32(int32_t x, int e) {
	uint32_t mask = ((uint32_t)1 << e) - 1u;
	uint32_t rem = (uint32_t)x & mask;
	uint32_t thr = (mask >> 1) + (x < 0 ? 1u : 0u);
	return (x >> e) + (rem > thr ? 1 : 0);
}

// src/intmath.cpp:244-251 (int64 instance), e in [0,63]
SSLM_HD int64_t rdbpot64(int64_t x, int e) {
	uint64_t mask = ((uint64_t)1 << e) - 1u;
	uint64_t rem = (uint64_t)x & mask;
	uint64_t thr = (mask >> 1) + (x < 0 ? 1u : 0u);
	return (x >> e) + (rem > thr ? 1 : 0);
}

// src/intmath.cpp:265-268 composed with forward_sites.cpp:461-470 (WSC1 fold: identity passes
// the accumulator through, otherwise MBQM of its int32 truncation).
SSLM_HD int64_t apply_fold(int64_t acc, int32_t identity, int32_t mult, int32_t shift) {
	if (identity != 0) return acc;
	return (int64_t)rdbpot32(srdhm((int32_t)acc, mult), shift);
}

// apply_fold for |acc| <= 2^29 (an int8 GEMM accumulator over K <= 32768), with the shift's
// rounding constants prepared per column by fold_consts: there srdhm cannot saturate
// (|acc * mult| < 2^60), and x / 2^s with ties away from zero is (x + 2^(s-1) - [x < 0]) >> s
// for s > 0 (|x| <= 2^29, so the sum stays in int32).
struct FoldConsts {
	int32_t mult, shift, half, nmask, identity;
};
SSLM_HD FoldConsts fold_consts(int32_t identity, int32_t mult, int32_t shift) {
	FoldConsts c;
	c.mult = mult;
	c.shift = shift;
	c.half = shift > 0 ? (int32_t)(1u << (shift - 1)) : 0;
	c.nmask = shift > 0 ? -1 : 0;
	c.identity = identity;
	return c;
}
SSLM_HD int32_t fold_bounded(int32_t acc, const FoldConsts& c) {
	const int32_t hi = (int32_t)(((int64_t)acc * c.mult + ((int64_t)1 << 30)) >> 31);
	const int32_t folded = (hi + c.half + ((hi >> 31) & c.nmask)) >> c.shift;
	return c.identity != 0 ? acc : folded;
}

// src/intmath.cpp:270-277
SSLM_HD int32_t sat_shl32(int32_t x, int shift) {
	if (shift <= 0) return x;
	int64_t w = (int64_t)x << shift;
	if (w > kI32Max) return kI32Max;
	if (w < kI32Min) return kI32Min;
	return (int32_t)w;
}

// forward_sites.cpp:472-481
SSLM_HD int64_t apply_amp_fold(int64_t acc, int32_t identity, int32_t mult, int32_t exponent) {
	if (identity != 0) return acc;
	int32_t hi = srdhm((int32_t)acc, mult);
	if (exponent >= 0) return (int64_t)rdbpot32(hi, exponent);
	return (int64_t)sat_shl32(hi, -exponent);
}

SSLM_HD int clz64(uint64_t n) { return n == 0 ? 64 : __builtin_clzll(n); }

// src/intmath.cpp:296-301
SSLM_HD int64_t normalize_scale(int64_t d_prime, int* s_out) {
	int p = 63 - clz64((uint64_t)d_prime);
	int s = 30 - p;
	*s_out = s;
	return s >= 0 ? (d_prime << s) : (d_prime >> 1);
}

// src/intmath.cpp:303-333 -- 3 Newton steps from a minimax seed, 2 correction steps.
SSLM_COLD int64_t reciprocal(int64_t dn) {
	const int64_t c32 = (2 * ((int64_t)48 << 31) + 17) / 34;
	const int64_t c32_2 = (2 * ((int64_t)32 << 31) + 17) / 34;
	int64_t y = c32 - ((c32_2 * dn) >> 31);
	for (int i = 0; i < 3; ++i) {
		int64_t dn_y = (int64_t)(((s128)dn * (s128)y) >> 31);
		int64_t delta = ((int64_t)1 << 32) - dn_y;
		y = (int64_t)(((s128)y * (s128)delta) >> 31);
	}
	for (int i = 0; i < 2; ++i) {
		s128 res2 = ((s128)((int64_t)1 << 62) - (s128)y * (s128)dn) * 2;
		if (res2 >= (s128)dn) {
			y += 1;
		} else if (res2 < -(s128)dn) {
			y -= 1;
		}
	}
	return y;
}

// Exact floor(n / d) for 0 <= n < 2^63, d >= 1: a double-precision estimate (off by at most one
// for these magnitudes) corrected with exact 128-bit residue checks.  Replaces the long 64-bit
// integer division sequence on the GPU; the result is the integer quotient bit for bit.
SSLM_COLD int64_t div_i64_cold(int64_t n, int64_t d) { return n / d; }

SSLM_HD int64_t div_floor_pos(int64_t n, int64_t d) {
	int64_t q = (int64_t)((double)n / (double)d);
	if (q >= ((int64_t)1 << 51)) return div_i64_cold(n, d);  // estimate no longer within one of the quotient
	if (q < 0) q = 0;
	s128 r = (s128)n - (s128)q * d;
	if (r < 0) {
		--q;
		r += d;
	}
	if (r < 0) {
		--q;
		r += d;
	}
	if (r >= d) {
		++q;
		r -= d;
	}
	if (r >= d) ++q;
	return q;
}

// round_half_up(2^62 / dn) for a canonical dn in [2^30, 2^31) -- the value the reference's
// corrected-Newton DynamicScaleReciprocal returns on that domain (src/intmath.cpp:303-333; its
// contract, include/superslm/intmath.h:124-131, is correct rounding over the whole normalized
// domain) -- from a correctly rounded double quotient and the reference's correction rule.
SSLM_HD int64_t reciprocal_div(int64_t dn) {
	int64_t y = (int64_t)(4611686018427387904.0 / (double)dn);
	for (int i = 0; i < 2; ++i) {  // the reference's correction rule: -dn <= 2(2^62 - y dn) < dn
		// y is within a few units of 2^62 / dn < 2^32, so y * dn < 2^63 and the residue is small:
		// 64-bit arithmetic is exact here
		const int64_t res2 = (((int64_t)1 << 62) - y * dn) * 2;
		if (res2 >= dn) {
			y += 1;
		} else if (res2 < -dn) {
			y -= 1;
		}
	}
	return y;
}

SSLM_HD int64_t reciprocal_norm(int64_t dn);

// reciprocal_div on the normalized domain (reciprocal_norm on the GPU: the same values, by an
// exhaustive check); outside it the reference recurrence itself is replayed.
SSLM_HD int64_t reciprocal_fast(int64_t dn) {
	if (dn < ((int64_t)1 << 30) || dn >= ((int64_t)1 << 31)) return reciprocal(dn);
#if defined(__HIP_DEVICE_COMPILE__)
	return reciprocal_norm(dn);
#else
	return reciprocal_div(dn);
#endif
}

// src/intmath.cpp:476-490 -- clamp(round_away(x*127*R / 2^(62-s)), +-127).
SSLM_HD int8_t requant_code(int64_t x, int64_t r, int s) {
	int exponent = 62 - s;
	uint64_t ax = x < 0 ? (~(uint64_t)x + 1u) : (uint64_t)x;
	u128 prod = (u128)ax * (uint64_t)r * 127u;
	u128 num = prod * 2 + ((u128)1 << exponent);
	uint64_t mag = (uint64_t)(num >> (exponent + 1));
	if (mag > 127u) mag = 127u;
	int32_t q = (int32_t)mag;
	return (int8_t)(x < 0 ? -q : q);
}

// Same composite for |x| <= 2^31 (the funnel's whole accepted domain): |x|*127*R < 2^70 is
// held as a (hi, lo) pair and the rounding shift 2^(62-s) (s in [-1, 30]) is done on 64-bit
// halves -- mag = (prod + 2^(e-1)) >> e is the reference's (2 prod + 2^e) >> (e + 1).
SSLM_HD int8_t requant_code_small(int64_t x, uint64_t r, int s) {
	const int e = 62 - s;  // 32..63
	const uint64_t ax = x < 0 ? (uint64_t)0 - (uint64_t)x : (uint64_t)x;
	const uint64_t a = ax * 127u;  // < 2^39
	const uint64_t lo = a * r;
	uint64_t hi = (uint64_t)(((u128)a * r) >> 64);
	const uint64_t lo2 = lo + ((uint64_t)1 << (e - 1));
	hi += lo2 < lo ? 1u : 0u;
	uint64_t mag = (lo2 >> e) | (hi << (64 - e));
	if ((hi >> e) != 0 || mag > 127u) mag = 127u;
	const int32_t q = (int32_t)mag;
	return (int8_t)(x < 0 ? -q : q);
}

// requant_code_small in double arithmetic, for |x| <= 2^31 and a funnel plan's (r, s), r in
// (2^31, 2^32] and s in [-1, 30].  The code is floor(q + 1/2), clamped to 127, for the exact
// quotient q = |x| 127 r / 2^(62-s).  f = 127 r 2^-(62-s) is exact in a double (127 r < 2^39),
// so |x| f is q rounded once and fma returns that rounding error exactly.  Rounding is
// monotone, so m0 = floor(rounded q + 1/2) is the code or one more; it is one more exactly when
// (rounded q - (m0 - 1/2)) + err < 0, a sign that is exact wherever it can be near zero
// (Sterbenz: there the rounded q is within 2^-40 of m0 - 1/2 >= 1/2).  Every operation is full
// rate on CDNA's FP64 pipes, where the 128-bit integer form takes eight quarter-rate multiplies.
SSLM_HD double requant_factor(int64_t r, int s) { return ldexp((double)(r * 127), -(62 - s)); }
SSLM_HD int8_t requant_code_f(int64_t x, double f) {
#pragma clang fp contract(off)
	const uint32_t ax = x < 0 ? 0u - (uint32_t)x : (uint32_t)x;
	const double a = (double)ax;
	const double qh = a * f;
	const double er = fma(a, f, -qh);
	const double q = fmin(qh, 255.0);  // past 255 the code saturates whatever the error
	const double m0 = floor(q + 0.5);
	const double m = (q - (m0 - 0.5)) + er < 0.0 ? m0 - 1.0 : m0;
	const int32_t c = (int32_t)fmin(m, 127.0);
	return (int8_t)(x < 0 ? -c : c);
}

// src/intmath.cpp:502-524
SSLM_HD int64_t isqrt(int64_t n) {
	int64_t rem = n, root = 0, bit = (int64_t)1 << 62;
	for (int i = 0; i < 32; ++i) {
		int64_t trial = root + bit;
		if (rem >= trial) {
			rem -= trial;
			root = (root >> 1) + bit;
		} else {
			root >>= 1;
		}
		bit >>= 2;
	}
	return root;
}

// floor(sqrt(n)) -- the value isqrt() returns for every int64 n (0 for n <= 0) -- from a
// double-precision estimate corrected with exact 64-bit squares.
// The double estimate is within one of floor(sqrt(n)) for every int64 n (n rounds to a double by
// at most 2^10, which moves the root by far less than one; the root rounds by at most 2^-21), so
// two fixed correction steps each way replace the loops (no loop: straight-line code on the GPU;
// (r + 1)^2 <= 3037000500^2 < 2^64 cannot wrap).
SSLM_HD int64_t isqrt_fast(int64_t n) {
	const uint64_t un = n > 0 ? (uint64_t)n : 0;
	uint64_t r = (uint64_t)sqrt((double)un);
#pragma unroll
	for (int i = 0; i < 2; ++i) r -= r * r > un ? 1 : 0;
#pragma unroll
	for (int i = 0; i < 2; ++i) r += (r + 1) * (r + 1) <= un ? 1 : 0;
	return (int64_t)r;
}

SSLM_HD int64_t sat_add64(int64_t a, int64_t b) {
	int64_t out = (int64_t)((uint64_t)a + (uint64_t)b);
	bool ovf = ((a >= 0) == (b >= 0)) && ((out >= 0) != (a >= 0));
	if (!ovf) return out;
	return a >= 0 ? kI64Max : kI64Min;
}

SSLM_HD int64_t sat_sub64(int64_t a, int64_t b) {
	int64_t out = (int64_t)((uint64_t)a - (uint64_t)b);
	bool ovf = ((a >= 0) != (b >= 0)) && ((out >= 0) != (a >= 0));
	if (!ovf) return out;
	return a >= 0 ? kI64Max : kI64Min;
}

// checked_chain_funnel.cpp:157-180
SSLM_HD Scale combine_scale(Scale a, Scale b) {
	int64_t e = sat_add64(sat_add64(a.e, b.e), 31);
	int64_t m = srdhm((int32_t)a.m, (int32_t)b.m);
	if (m < ((int64_t)1 << 30)) {
		m <<= 1;
		e -= 1;
	}
	return Scale{m, e};
}

SSLM_HD bool fits_i32(int64_t v) { return v >= kI32Min && v <= kI32Max; }

// Reference forward status codes (include/superslm/checked_chain_funnel.h:68-284, same order).
enum FwdStatus : int32_t {
	kOk = 0,
	kChainInputOutOfDomain = 1,
	kLogitNarrowingOverflow = 2,
	kIExpConstantsOutOfDomain = 3,
	kCarriedScaleMantissaOutOfDomain = 4,
	kSiluCompositionScaleOutOfDomain = 5,
	kRdbpotExponentOutOfDomain = 6,
	kSoftmaxRowWidthOutOfDomain = 7,
	kTokenIdOutOfRange = 8,
	kPositionOverCap = 9,
	kSoftmaxKernelRefusedAfterGateAccepted = 20,
	kResidualReconciliationMagnitudeOutOfDomain = 21,
	kIExpScaleDerivationOutOfDomain = 23,
	kBiasReconcileProductOutOfDomain = 24,
};

// The funnel's scale half (checked_chain_funnel.cpp:268-329): checks, the D'-derived (Dn, s, R)
// and the left-associated fold of incoming factors, the site constant and (Dn, -s).
// `d_prime` is the row's max |x| with the all-zero guard applied.  Returns a status; on Ok the
// per-element codes are requant_code_small(x, r, s).
struct FunnelPlan {
	int64_t r;
	int s;
	Scale out;
};

struct FunnelOut {
	int32_t st;
	int32_t s;
	int64_t r;
	Scale out;
};

// reciprocal_div for a normalized dn in [2^30, 2^31), the only divisors a funnel plan has.  On the
// GPU the estimate of 2^62 / dn is the hardware double reciprocal refined by one Newton step
// (relative error near 2^-50, so within one of the quotient, which lies in (2^31, 2^32]) and
// converted with one unsigned 32-bit conversion (it saturates at 2^32 - 1 only for dn = 2^30,
// which the first correction step lifts to 2^32); the reference's two correction steps follow.
// Checked equal to reciprocal_div for every dn in [2^30, 2^31) by tests/reciprocal_norm_check.
SSLM_HD int64_t reciprocal_norm(int64_t dn) {
#if defined(__HIP_DEVICE_COMPILE__)
	const double dd = (double)dn;
	double r = __builtin_amdgcn_rcp(dd);
	r = fma(r, fma(-dd, r, 1.0), r);
	int64_t y = (int64_t)__double2uint_rz(4611686018427387904.0 * r);
	for (int i = 0; i < 2; ++i) {
		const int64_t res2 = (((int64_t)1 << 62) - y * dn) * 2;
		y += res2 >= dn ? 1 : (res2 < -dn ? -1 : 0);
	}
	return y;
#else
	return reciprocal_div(dn);
#endif
}

// By-value form with at most two incoming factors.  Inlined: in the row kernels its inputs are
// wave-uniform, so it compiles to scalar code.  Every part is computed and the status is chosen
// at the end, in the reference's order (the incoming and site mantissas, then D', then the folds):
// without early returns the reciprocal and the scale folds interleave (a dependent chain of plans
// took 318 ns each with them, 198 ns without and with reciprocal_norm).
SSLM_HD FunnelOut funnel_plan_v(uint64_t d_prime, int n_in, Scale in0, Scale in1, Scale site) {
	const bool ok_in = !((n_in > 0 && !fits_i32(in0.m)) || (n_in > 1 && !fits_i32(in1.m))) && fits_i32(site.m);
	const uint64_t d = d_prime < 1 ? 1 : d_prime;
	const bool ok_d = d <= ((uint64_t)1 << 31);
	int s;
	const int64_t dn = normalize_scale((int64_t)(ok_d ? d : 1), &s);
	const int64_t r = reciprocal_norm(dn);
	Scale run = site;
	bool ok_mid = true;
	if (n_in > 0) {
		run = in0;
		if (n_in > 1) {
			run = combine_scale(run, in1);
			ok_mid = fits_i32(run.m);
		}
		run = combine_scale(run, site);
	}
	const bool ok1 = fits_i32(run.m);
	run = combine_scale(run, Scale{dn, -(int64_t)s});
	const bool ok2 = fits_i32(run.m);
	FunnelOut o{};
	o.st = !ok_in ? kCarriedScaleMantissaOutOfDomain
	              : (!ok_d ? kChainInputOutOfDomain : (ok_mid && ok1 && ok2 ? kOk : kCarriedScaleMantissaOutOfDomain));
	o.s = s;
	o.r = r;
	o.out = run;
	return o;
}

// n_in <= 2 (every site of the forward path)
SSLM_HD int32_t funnel_plan(uint64_t d_prime, const Scale* incoming, int n_in, Scale site, FunnelPlan* plan) {
	const Scale z{0, 0};
	const FunnelOut o = funnel_plan_v(d_prime, n_in, n_in > 0 ? incoming[0] : z, n_in > 1 ? incoming[1] : z, site);
	if (o.st == kOk) {
		plan->r = o.r;
		plan->s = o.s;
		plan->out = o.out;
	}
	return o.st;
}

// forward_sites.cpp:389-395
SSLM_HD int64_t composed_exponent(int64_t e_a, int64_t e_t) {
	int64_t k = sat_sub64(62, sat_sub64(e_a, e_t));
	if (k > 4096) k = 4096;
	if (k < -4096) k = -4096;
	return k;
}

// forward_sites.cpp:513-653 -- round_away(branch*m_a*r_t / 2^k), k = 62-(e_a-e_t); a negative k
// is an exact left shift.  *clamped: the saturation-counter predicate; *exceeded: the true
// magnitude does not fit int64.
SSLM_HD int64_t landing_rescale(int64_t branch, int64_t m_a, int64_t r_t, int64_t k, bool* clamped,
                                 bool* exceeded) {
	bool neg = (branch < 0) != (m_a < 0);
	uint64_t ab = branch < 0 ? (~(uint64_t)branch + 1u) : (uint64_t)branch;
	uint64_t am = m_a < 0 ? (~(uint64_t)m_a + 1u) : (uint64_t)m_a;
	u128 mag = (u128)ab * am * (uint64_t)r_t;
	int64_t raw;
	bool exc_clamp, exc_i64;
	if (k >= 0) {
		u128 doubled = mag + mag;
		u128 one_k = k >= 128 ? (u128)0 : ((u128)1 << k);
		u128 q = (k + 1 >= 128) ? (u128)0 : ((doubled + one_k) >> (k + 1));
		uint64_t qhi = (uint64_t)(q >> 64), qlo = (uint64_t)q;
		exc_clamp = (qhi != 0) || qlo > 127;
		exc_i64 = (qhi != 0) || qlo > (uint64_t)kI64Max;
		raw = (int64_t)qlo;
	} else {
		int sh = (int)(-k);
		u128 shifted = sh >= 128 ? (u128)0 : (mag << sh);
		if (sh >= 128) {
			exc_clamp = mag != 0;
			exc_i64 = exc_clamp;
		} else {
			bool lost = (shifted >> sh) != mag;
			uint64_t shi = (uint64_t)(shifted >> 64), slo = (uint64_t)shifted;
			exc_clamp = lost || shi != 0 || slo > 127;
			exc_i64 = lost || shi != 0 || slo > (uint64_t)kI64Max;
		}
		raw = (int64_t)(uint64_t)shifted;
	}
	if (neg) raw = (int64_t)(0u - (uint64_t)raw);
	*clamped = exc_clamp || raw < -127 || raw > 127;
	*exceeded = exc_i64;
	return raw;
}

struct Landing {
	int64_t raw;
	bool clamped, exceeded;
};

SSLM_COLD Landing landing_rescale_cold(int64_t branch, int64_t m_a, int64_t r_t, int64_t k) {
	Landing l;
	l.raw = landing_rescale(branch, m_a, r_t, k, &l.clamped, &l.exceeded);
	return l;
}

// landing_rescale for the residual site's operands (|branch| <= 127 code, |m_a| < 2^31 + 1,
// r_t < 2^33) on 64-bit halves when the composed exponent k is non-negative; every other case
// takes the general 128-bit path above.  Same outputs bit for bit.
SSLM_HD int64_t landing_small(int64_t branch, int64_t m_a, int64_t r_t, int64_t k, bool* clamped, bool* exceeded) {
	const uint64_t ab = branch < 0 ? (uint64_t)0 - (uint64_t)branch : (uint64_t)branch;
	const uint64_t am = m_a < 0 ? (uint64_t)0 - (uint64_t)m_a : (uint64_t)m_a;
	if (k < 0 || ab > 127u || am > ((uint64_t)1 << 31) || (uint64_t)r_t >= ((uint64_t)1 << 33))
	{
		const Landing l = landing_rescale_cold(branch, m_a, r_t, k);
		*clamped = l.clamped;
		*exceeded = l.exceeded;
		return l.raw;
	}
	const bool neg = (branch < 0) != (m_a < 0);
	const uint64_t a = ab * am;  // < 2^39
	const uint64_t lo = a * (uint64_t)r_t;
	const uint64_t hi = (uint64_t)(((u128)a * (uint64_t)r_t) >> 64);  // prod < 2^72
	uint64_t qlo, qhi;
	if (k == 0) {
		qlo = lo;
		qhi = hi;
	} else if (k >= 73) {
		qlo = 0;
		qhi = 0;
	} else {
		// (prod + 2^(k-1)) >> k
		uint64_t alo = lo, ahi = hi;
		if (k - 1 < 64) {
			alo = lo + ((uint64_t)1 << (k - 1));
			ahi = hi + (alo < lo ? 1u : 0u);
		} else {
			ahi = hi + ((uint64_t)1 << (k - 1 - 64));
		}
		if (k < 64) {
			qlo = (alo >> k) | (ahi << (64 - k));
			qhi = ahi >> k;
		} else {
			qlo = ahi >> (k - 64);
			qhi = 0;
		}
	}
	const bool exc_clamp = qhi != 0 || qlo > 127;
	const bool exc_i64 = qhi != 0 || qlo > (uint64_t)kI64Max;
	int64_t raw = (int64_t)qlo;
	if (neg) raw = (int64_t)(0u - (uint64_t)raw);
	*clamped = exc_clamp || raw < -127 || raw > 127;
	*exceeded = exc_i64;
	return raw;
}

SSLM_HD int64_t clamp_code(int64_t v) { return v > 127 ? 127 : (v < -127 ? -127 : v); }

// forward_sites.cpp:399-408
SSLM_HD int64_t floor_div(int64_t a, int64_t b) {
	int64_t q = a / b, r = a % b;
	return (r != 0 && r < 0) ? q - 1 : q;
}

// src/intmath.cpp:782-792
SSLM_HD void rope_pair(int32_t x, int32_t y, int32_t c, int32_t s, int64_t* ox, int64_t* oy) {
	int64_t xr = (int64_t)x * c - (int64_t)y * s;
	int64_t yr = (int64_t)x * s + (int64_t)y * c;
	*ox = rdbpot64(xr, 30);
	*oy = rdbpot64(yr, 30);
}

// src/silu_lut.cpp:16-67
SSLM_HD int32_t silu_sigmoid_q15(const int32_t* table, int8_t code, int64_t m, int e) {
	int64_t term = (int64_t)code * m;
	int shift = e + 5 + 12;
	int64_t pos = shift >= 0 ? (term << shift) : rdbpot64(term, -shift);
	const int64_t hi_dom = (int64_t)1024 << 12;
	pos += hi_dom / 2;
	if (pos < 0) pos = 0;
	else if (pos > hi_dom) pos = hi_dom;
	int64_t i0 = pos >> 12;
	if (i0 > 1023) i0 = 1023;
	int64_t frac = pos - (i0 << 12);
	int64_t lo = table[i0], hi = table[i0 + 1];
	return (int32_t)(lo + rdbpot64(frac * (hi - lo), 12));
}

// checked_chain_funnel.cpp:402-405, 484-499
SSLM_HD int32_t check_silu_scale(int64_t m, int64_t e) {
	const int64_t max_abs_m = ((int64_t)1 << 31) - 1;
	if (m < -max_abs_m || m > max_abs_m) return kSiluCompositionScaleOutOfDomain;
	if (e < -80 || e > 8) return kSiluCompositionScaleOutOfDomain;
	return kOk;
}

// src/intmath.cpp:702-778 -- the C30 derivation of the i-exp triple from a carried scale.
// Returns 0 on success (the reference's kOk), non-zero for every rejection.
SSLM_HD int iexp_scale_constants(int64_t m, int64_t e, int64_t ln2_q, int64_t b_q, int64_t ca_q, int64_t* q_ln2,
                                 int64_t* q_b, int64_t* q_c) {
	const int fmt = 30;
	if (ln2_q <= 0 || b_q <= 0 || ca_q <= 0) return 1;
	int64_t sh_ln2 = sat_add64(sat_add64(fmt, 62), e);
	int64_t sh_b = sat_add64(sat_add64(fmt, 62), e);
	int64_t sh_c = sat_add64(sat_add64(fmt, 124), sat_add64(e, e));
	int64_t mn = sh_ln2 < sh_b ? sh_ln2 : sh_b;
	if (sh_c < mn) mn = sh_c;
	if (mn < 0) return 2;
	uint64_t r = (uint64_t)reciprocal_fast(m);
	u128 n_ln2 = (u128)(uint64_t)ln2_q * r;
	u128 n_b = (u128)(uint64_t)b_q * r;
	u128 n_c = (u128)r * r * (uint64_t)ca_q;
	u128 f_ln2 = sh_ln2 >= 128 ? (u128)0 : (n_ln2 >> sh_ln2);
	u128 f_b = sh_b >= 128 ? (u128)0 : (n_b >> sh_b);
	u128 f_c = sh_c >= 128 ? (u128)0 : (n_c >> sh_c);
	if (f_ln2 > (u128)kI64Max || f_b > (u128)kI64Max || f_c > (u128)kI64Max) return 3;
	*q_ln2 = (int64_t)f_ln2;
	*q_b = (int64_t)f_b;
	*q_c = (int64_t)f_c;
	return 0;
}

// checked_chain_funnel.cpp:520-583
SSLM_HD int32_t check_softmax_width(int64_t q_b, int64_t q_c, int64_t width) {
	if (q_c < 0) return kSoftmaxRowWidthOutOfDomain;
	if (width <= 0) return kSoftmaxRowWidthOutOfDomain;
	s128 m128 = (s128)q_b * q_b + (s128)q_c;
	if (m128 > (s128)kI64Max || m128 > (s128)kSoftmaxMaxSafe) return kSoftmaxRowWidthOutOfDomain;
	int64_t m = (int64_t)m128;
	// width > floor(INT64_MAX / m)  <=>  width * m > INT64_MAX  (width, m >= 1): no 64-bit division
	if (m != 0 && (u128)(uint64_t)width * (uint64_t)m > (u128)kI64Max) return kSoftmaxRowWidthOutOfDomain;
	return kOk;
}

// src/intmath.cpp:580-668 + :540-567 for one softmax element (intmath.cpp:859-888): returns
// the i-exp value, or -1 when the element is refused (a kBad* construction, or a value outside
// [0, M]).  `shifted` = score - row max (<= 0 always, so kBadQ never fires).
SSLM_HD int64_t iexp_element(int64_t shifted, int64_t q_ln2, int64_t q_b, int64_t q_c, int64_t m_ceiling) {
	const int64_t max_qln2 = kI64Max / 30;
	if (shifted > 0) return -1;
	if (q_ln2 < 1 || q_ln2 > max_qln2) return -1;
	int64_t clip_lo = -30 * q_ln2;
	int64_t clipped = shifted < clip_lo ? clip_lo : shifted;
	int64_t z = div_floor_pos(-clipped, q_ln2);
	int64_t q_p = clipped + z * q_ln2;
	if (q_b < kI64Min - q_p) return -1;
	int64_t base = q_p + q_b;
	s128 v = (s128)base * base + (s128)q_c;
	int64_t value = (int64_t)(v >> z);
	if (m_ceiling <= 0 || value < 0 || value > m_ceiling) return -1;
	return value;
}

// floor(n / d) for 0 <= n, 1 <= d, given inv = 1.0 / d and that the true quotient lies in
// [0, qmax] with qmax * d + d < 2^63: the double estimate is exact to within one for quotients
// far below 2^50 and is corrected with exact 64-bit remainders.
SSLM_HD int64_t div_rcp(int64_t n, int64_t d, double inv, int64_t qmax) {
	int64_t q = (int64_t)((double)n * inv);
	q = q < 0 ? 0 : (q > qmax ? qmax : q);
	int64_t r = n - q * d;
	while (r < 0) {
		--q;
		r += d;
	}
	while (r >= d) {
		++q;
		r -= d;
	}
	return q;
}

// iexp_element (intmath.cpp:580-668) for a row whose constants passed check_softmax_width
// (q_c >= 0, q_b^2 + q_c <= kSoftmaxMaxSafe) and shifted <= 0:
// the quotient z in [0, 30] from a reciprocal, and the square in 64 bits when |base| < 2^31
// (then base^2 + q_c < 2^63); the 128-bit form otherwise.  Same value, or -1 when refused.
SSLM_HD int64_t iexp_fast(int64_t shifted, int64_t q_ln2, double inv_ln2, int64_t q_b,
                                             int64_t q_c, int64_t m_ceiling) {
	if (q_ln2 < 1 || q_ln2 > kI64Max / 30) return -1;
	const int64_t x = shifted < -30 * q_ln2 ? 30 * q_ln2 : -shifted;
	int64_t z = (int64_t)((double)x * inv_ln2);
	z = z < 0 ? 0 : (z > 30 ? 30 : z);
	int64_t r = x - z * q_ln2;  // q_p = -r
	while (r < 0) {
		--z;
		r += q_ln2;
	}
	while (r >= q_ln2) {
		++z;
		r -= q_ln2;
	}
	if (q_b < kI64Min + r) return -1;
	const int64_t base = q_b - r;
	int64_t value;
	if (base > -(int64_t(1) << 31) && base < (int64_t(1) << 31)) value = (base * base + q_c) >> z;
	else value = (int64_t)((((s128)base * base) + (s128)q_c) >> z);
	if (m_ceiling <= 0 || value < 0 || value > m_ceiling) return -1;
	return value;
}

// The softmax's per-element ceiling M = q_b^2 + q_c when usable (intmath.cpp:831-851), else 0.
// iexp_fast on 32-bit operands, for a row whose constants pass iexp_small_ok (and the width
// gate: q_c >= 0, q_b^2 + q_c <= kSoftmaxMaxSafe): then x, z, r and base = q_b - r fit int32
// and base^2 + q_c is one 32 x 32 + 64-bit multiply-add; same value, or -1 when refused.
SSLM_HD bool iexp_small_ok(int64_t q_ln2, int64_t q_b, int64_t m_ceiling) {
	const int64_t ab = q_b < 0 ? -q_b : q_b;
	return q_ln2 >= 1 && q_ln2 <= kI32Max / 30 && ab <= kI32Max - q_ln2 && m_ceiling > 0;
}
// iexp_small in two halves: the quotient z = floor(x / q_ln2) and remainder r of x = -shifted
// (clipped at 30 q_ln2), packed as z << 27 | r (r < q_ln2 <= 2^31 / 30 < 2^27, z <= 30), then the
// value from them -- so a caller may keep the 32-bit pair and finish the value later.
SSLM_HD uint32_t iexp_small_zr(int64_t shifted, int32_t q_ln2, double inv_ln2) {
	const int32_t lim = 30 * q_ln2;
	const int32_t x = shifted < -(int64_t)lim ? lim : (int32_t)(-shifted);
	// x / q_ln2 <= 30 and the double estimate is within 30 * 2^-52 of it, while a quotient that
	// is not an integer is at least 1 / q_ln2 >= 2^-31 below the next one: the truncation is
	// floor(x / q_ln2) or, for an exact quotient estimated low, one less.  One corrective step
	// each way (selects, no loop) therefore gives the exact quotient and remainder.
	int32_t z = (int32_t)((double)x * inv_ln2);
	z = z < 0 ? 0 : (z > 30 ? 30 : z);
	int32_t r = x - z * q_ln2;
	const bool lo = r < 0;
	z = lo ? z - 1 : z;
	r = lo ? r + q_ln2 : r;
	const bool hi = r >= q_ln2;
	z = hi ? z + 1 : z;
	r = hi ? r - q_ln2 : r;
	return (uint32_t)z << 27 | (uint32_t)r;
}
SSLM_HD int64_t iexp_small_value(uint32_t zr, int32_t q_b, int64_t q_c, int64_t m_ceiling) {
	const int32_t base = q_b - (int32_t)(zr & ((1u << 27) - 1u));
	const uint32_t ab = base < 0 ? 0u - (uint32_t)base : (uint32_t)base;
	const uint64_t v = ((uint64_t)ab * ab + (uint64_t)q_c) >> (zr >> 27);
	return v > (uint64_t)m_ceiling ? -1 : (int64_t)v;
}
SSLM_HD int64_t iexp_small(int64_t shifted, int32_t q_ln2, double inv_ln2, int32_t q_b, int64_t q_c,
                           int64_t m_ceiling) {
	return iexp_small_value(iexp_small_zr(shifted, q_ln2, inv_ln2), q_b, q_c, m_ceiling);
}

// The Q15 probability floor((e << 15) / d) for 0 <= e <= d < 2^38 in doubles: e 2^15 and d are
// exact, the estimate n / d is off by less than 2^-37, and fma gives the remainder n - q d
// exactly, so one step corrects it (div_floor_pos's value).
SSLM_HD bool div_q15_small_ok(int64_t d) { return d >= 1 && d < ((int64_t)1 << 38); }
SSLM_HD int32_t div_q15_small(int64_t e, double d, double inv) {
#pragma clang fp contract(off)
	const double n = (double)e * 32768.0;
	double q = fmin(trunc(n * inv), 32768.0);
	const double r = fma(-q, d, n);
	q = r < 0.0 ? q - 1.0 : (r >= d ? q + 1.0 : q);
	return (int32_t)q;
}

// floor(v 2^32 / root) for a code v in [-128, 127] and 1 <= root < 2^24 (the RMSNorm's
// per-code quotient, forward_sites.cpp:410-459: floor for v >= 0, -ceil(|v| 2^32 / root) below),
// given inv = 1.0 / root.  n = |v| 2^32 <= 2^39 is exact in a double and the estimate n inv is
// within one of the quotient; q root <= n + root < 2^53 is exact too, so fma gives the exact
// remainder for the one-step correction.
SSLM_HD int64_t norm_fd(int32_t v, double root, double inv) {
	const double n = ldexp((double)(v < 0 ? -v : v), 32);
	double q = floor(n * inv);
	double r = fma(-q, root, n);
	if (r < 0.0) {
		q -= 1.0;
		r += root;
	} else if (r >= root) {
		q += 1.0;
		r -= root;
	}
	const int64_t qi = (int64_t)q;
	return v >= 0 ? qi : -(qi + (r > 0.0 ? 1 : 0));
}

SSLM_HD int64_t softmax_ceiling(int64_t q_b, int64_t q_c) {
	s128 m128 = (s128)q_b * q_b + (s128)q_c;
	bool usable = m128 <= (s128)kI64Max && m128 >= 1 && m128 <= (s128)kSoftmaxMaxSafe;
	return usable ? (int64_t)m128 : 0;
}

// src/intmath.cpp:381-418 + checked_chain_funnel.cpp:454-482: the bias term
// round_away(b*r_a / 2^(30+62+e_a)); false when the exponent or the sum with `acc` is out of
// domain.
// The general form on 128-bit products (any bias code).  Returns its result by value (an
// out-of-line call given a pointer would keep the caller's variable in scratch memory).
struct BiasTerm {
	int64_t term;
	bool ok;
};

SSLM_COLD BiasTerm bias_term_wide(int64_t b, int64_t r_a, int64_t e_a, int64_t acc) {
	BiasTerm r{0, false};
	s128 sum = (s128)30 + 62 + (s128)e_a;
	if (sum < 0 || sum > 63) return r;
	int exponent = (int)sum;
	s128 wide = (s128)b * (s128)r_a;
	uint64_t mask = ((uint64_t)1 << exponent) - 1u;
	uint64_t rem = (uint64_t)wide & mask;
	uint64_t thr = (mask >> 1) + (wide < 0 ? 1u : 0u);
	s128 rounded = (wide >> exponent) + (rem > thr ? 1 : 0);
	if (rounded != (s128)(int64_t)rounded) return r;
	int64_t term = (int64_t)rounded;
	uint64_t s = (uint64_t)acc + (uint64_t)term;
	if (((((uint64_t)acc ^ (uint64_t)term) >> 63) == 0) && ((((uint64_t)acc ^ s) >> 63) != 0)) return r;
	r.term = term;
	r.ok = true;
	return r;
}

// Same result; |b| < 2^30 with 0 <= r_a <= 2^33 (every bias of a real artifact against a
// reciprocal of a canonical mantissa) keeps b * r_a inside int64, so the common case needs no
// 128-bit arithmetic.
SSLM_HD bool bias_term(int64_t b, int64_t r_a, int64_t e_a, int64_t acc, int64_t* out) {
	const uint64_t ab = b < 0 ? (uint64_t)0 - (uint64_t)b : (uint64_t)b;
	if (ab >= ((uint64_t)1 << 30) || r_a < 0 || r_a > ((int64_t)1 << 33)) {
		const BiasTerm w = bias_term_wide(b, r_a, e_a, acc);
		if (w.ok) *out = w.term;
		return w.ok;
	}
	if (e_a < -92 || e_a > -29) return false;  // exponent 92 + e_a outside [0, 63]
	const int exponent = (int)(92 + e_a);
	const int64_t wide = b * r_a;
	const uint64_t mask = ((uint64_t)1 << exponent) - 1u;
	const uint64_t rem = (uint64_t)wide & mask;
	const uint64_t thr = (mask >> 1) + (wide < 0 ? 1u : 0u);
	const int64_t term = (wide >> exponent) + (rem > thr ? 1 : 0);
	const uint64_t s = (uint64_t)acc + (uint64_t)term;
	if (((((uint64_t)acc ^ (uint64_t)term) >> 63) == 0) && ((((uint64_t)acc ^ s) >> 63) != 0)) return false;
	*out = term;
	return true;
}

}  // namespace sslm
