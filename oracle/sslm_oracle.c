/* CPU restatement of SuperSLM's integer forward path -- TEST INFRASTRUCTURE ONLY.
 * See sslm_oracle.h for what may load this file and how it is pinned.  Every definition cites
 * the reference file:line whose behaviour it restates (paths relative to the reference root). */
#include "sslm_oracle.h"

#include <stdlib.h>
#include <string.h>

typedef __int128 s128;
typedef unsigned __int128 u128;

#define I32_MIN (-2147483647 - 1)
#define I32_MAX 2147483647
#define I64_MAX 0x7fffffffffffffffLL
#define I64_MIN (-I64_MAX - 1)

/* ======================= primitives: src/intmath.cpp ======================= */

/* src/intmath.cpp:230-236 -- (a*b + 2^30) >> 31, floor shift, saturating only at INT32_MAX. */
int32_t or_srdhm(int32_t a, int32_t b) {
	int64_t ab = (int64_t)a * (int64_t)b;
	int64_t r = (ab + ((int64_t)1 << 30)) >> 31;
	return r > I32_MAX ? I32_MAX : (int32_t)r;
}

/* src/intmath.cpp:244-251 -- x / 2^e rounded half away from zero. */
int32_t or_rdbpot32(int32_t x, int exponent) {
	uint32_t mask = (exponent >= 32) ? 0xffffffffu : (((uint32_t)1 << exponent) - 1u);
	uint32_t rem = (uint32_t)x & mask;
	uint32_t thr = (mask >> 1) + (x < 0 ? 1u : 0u);
	return (x >> exponent) + (rem > thr ? 1 : 0);
}

int64_t or_rdbpot64(int64_t x, int exponent) {
	uint64_t mask = (((uint64_t)1 << exponent) - 1u);
	uint64_t rem = (uint64_t)x & mask;
	uint64_t thr = (mask >> 1) + (x < 0 ? 1u : 0u);
	return (x >> exponent) + (rem > thr ? 1 : 0);
}

/* src/intmath.cpp:265-268 */
int32_t or_mbqm(int32_t x, int32_t mult, int shift) { return or_rdbpot32(or_srdhm(x, mult), shift); }

/* src/intmath.cpp:270-277 */
int32_t or_sat_shl32(int32_t x, int shift) {
	if (shift <= 0) return x;
	int64_t w = (int64_t)x << shift;
	if (w > I32_MAX) return I32_MAX;
	if (w < I32_MIN) return I32_MIN;
	return (int32_t)w;
}

/* src/intmath.cpp:280-284 */
int or_clz64(uint64_t n) { return n == 0 ? 64 : __builtin_clzll(n); }

/* src/intmath.cpp:427-450 -- unsigned magnitude, all-zero guard, saturating narrow. */
int64_t or_max_abs_wide(const int64_t* x, size_t n) {
	uint64_t d = 0;
	for (size_t i = 0; i < n; ++i) {
		uint64_t a = x[i] < 0 ? (~(uint64_t)x[i] + 1u) : (uint64_t)x[i];
		if (a > d) d = a;
	}
	if (d < 1) d = 1;
	return d > (uint64_t)I64_MAX ? I64_MAX : (int64_t)d;
}

/* src/intmath.cpp:296-301 */
int64_t or_normalize_scale(int64_t d_prime, int* out_s) {
	int p = 63 - or_clz64((uint64_t)d_prime);
	int s = 30 - p;
	*out_s = s;
	return s >= 0 ? (d_prime << s) : (d_prime >> 1);
}

/* src/intmath.cpp:303-333 -- seed line, 3 Newton steps, 2 correction steps. */
int64_t or_reciprocal(int64_t dn) {
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

/* src/intmath.cpp:476-490 -- clamp(round_away(x*127*R / 2^(62-s)), +-127). */
int8_t or_requant_code_wide(int64_t x, int64_t r, int s) {
	int exponent = 62 - s;
	uint64_t ax = x < 0 ? (~(uint64_t)x + 1u) : (uint64_t)x;
	u128 prod = (u128)ax * (uint64_t)r * 127u;
	u128 num = prod * 2 + ((u128)1 << exponent);
	uint64_t mag = (uint64_t)(num >> (exponent + 1)); /* low 64 bits, as UShrToU64 */
	if (mag > 127u) mag = 127u;
	int32_t q = (int32_t)mag;
	return (int8_t)(x < 0 ? -q : q);
}

/* src/intmath.cpp:502-524 -- restoring square root, 32 unconditional digit steps. */
int64_t or_isqrt(int64_t n) {
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

/* src/intmath.cpp:580-668 -- returns 0 kOk, 1 kNotRepresentable, 2 kBadQ, 3 kBadQLn2, 4 kBadQB.
 * z/base are written for outcomes 0 and 1. */
int or_iexp_construct(int64_t q, int64_t q_ln2, int64_t q_b, int64_t q_c, int64_t* z_out,
                      int64_t* base_out) {
	const int64_t max_qln2 = I64_MAX / 30;
	if (q > 0) return 2;
	if (q_ln2 < 1 || q_ln2 > max_qln2) return 3;
	int64_t clip_lo = -30 * q_ln2;
	int64_t clipped = q < clip_lo ? clip_lo : q;
	int64_t z = (-clipped) / q_ln2;
	int64_t q_p = clipped + z * q_ln2;
	if (q_b < I64_MIN - q_p) return 4;
	int64_t base = q_p + q_b;
	if (z_out) *z_out = z;
	if (base_out) *base_out = base;
	s128 v = (s128)base * base + (s128)q_c;
	s128 limit = (s128)1 << (63 + z);
	return (v <= limit - 1 && v >= -limit) ? 0 : 1;
}

/* src/intmath.cpp:540-567 -- (base^2 + q_c) >> z, floor shift, low 64 bits. */
int64_t or_iexp_evaluate(int64_t z, int64_t base, int64_t q_c) {
	s128 v = (s128)base * base + (s128)q_c;
	return (int64_t)(v >> z);
}

static int64_t sat_add64(int64_t a, int64_t b) {
	int64_t out = (int64_t)((uint64_t)a + (uint64_t)b);
	int ovf = ((a >= 0) == (b >= 0)) && ((out >= 0) != (a >= 0));
	if (!ovf) return out;
	return a >= 0 ? I64_MAX : I64_MIN;
}

/* src/intmath.cpp:702-778 -- returns 0 kOk, 1 kBadCoefficient, 2 kNegativeShift,
 * 3 kNotRepresentable. */
int or_iexp_scale_constants(int64_t m, int64_t e, int64_t ln2_q, int ln2_fmt, int64_t b_q, int b_fmt,
                            int64_t ca_q, int ca_fmt, int64_t* q_ln2, int64_t* q_b, int64_t* q_c) {
	if (ln2_q <= 0 || b_q <= 0 || ca_q <= 0) return 1;
	int64_t sh_ln2 = sat_add64(sat_add64(ln2_fmt, 62), e);
	int64_t sh_b = sat_add64(sat_add64(b_fmt, 62), e);
	int64_t two_e = sat_add64(e, e);
	int64_t sh_c = sat_add64(sat_add64(ca_fmt, 124), two_e);
	int64_t mn = sh_ln2;
	if (sh_b < mn) mn = sh_b;
	if (sh_c < mn) mn = sh_c;
	if (mn < 0) return 2;
	uint64_t r = (uint64_t)or_reciprocal(m);
	u128 n_ln2 = (u128)(uint64_t)ln2_q * r;
	u128 n_b = (u128)(uint64_t)b_q * r;
	u128 n_c = (u128)r * r * (uint64_t)ca_q;
	u128 f_ln2 = sh_ln2 >= 128 ? 0 : (n_ln2 >> sh_ln2);
	u128 f_b = sh_b >= 128 ? 0 : (n_b >> sh_b);
	u128 f_c = sh_c >= 128 ? 0 : (n_c >> sh_c);
	if (f_ln2 > (u128)I64_MAX || f_b > (u128)I64_MAX || f_c > (u128)I64_MAX) return 3;
	if (q_ln2) *q_ln2 = (int64_t)f_ln2;
	if (q_b) *q_b = (int64_t)f_b;
	if (q_c) *q_c = (int64_t)f_c;
	return 0;
}

/* include/superslm/intmath.h:518-527 -- the format-30 coefficient triple, truncated from the
 * same doubles. */
void or_iexp_pinned(int64_t* ln2_q, int64_t* b_q, int64_t* ca_q) {
	const double ln2 = 0x1.62e42fefa39efp-1;
	*ln2_q = (int64_t)(ln2 * (double)((int64_t)1 << 30));
	*b_q = (int64_t)(1.353 * (double)((int64_t)1 << 30));
	*ca_q = (int64_t)((0.344 / 0.3585) * (double)((int64_t)1 << 30));
}

/* src/intmath.cpp:782-792 -- one rounding at 30 fractional bits, unclamped. */
void or_rope_pair(int32_t x, int32_t y, int32_t c, int32_t s, int64_t* ox, int64_t* oy) {
	int64_t xr = (int64_t)x * c - (int64_t)y * s;
	int64_t yr = (int64_t)x * s + (int64_t)y * c;
	*ox = or_rdbpot64(xr, 30);
	*oy = or_rdbpot64(yr, 30);
}

#define SOFTMAX_MAX_SAFE (((int64_t)1 << 62) >> 15) /* checked_chain_funnel.h:563 */

/* src/intmath.cpp:796-901 -- returns 1 when every element was well formed. */
int or_softmax_row_q15(const int64_t* scores, size_t width, int64_t q_ln2, int64_t q_b, int64_t q_c,
                       int64_t* out_probs) {
	if (width == 0) return 1;
	s128 m128 = (s128)q_b * q_b + (s128)q_c;
	int m_usable = m128 <= (s128)I64_MAX && m128 >= 1 && m128 <= (s128)SOFTMAX_MAX_SAFE;
	int64_t mx = m_usable ? (int64_t)m128 : 0;
	int64_t peak = scores[0];
	for (size_t i = 1; i < width; ++i)
		if (scores[i] > peak) peak = scores[i];
	int64_t* exps = (int64_t*)malloc(width * sizeof(int64_t));
	int64_t total = 0;
	int ok = 1;
	for (size_t k = 0; k < width; ++k) {
		int64_t z, base;
		int d = or_iexp_construct(scores[k] - peak, q_ln2, q_b, q_c, &z, &base);
		if (d >= 2) {
			ok = 0;
			exps[k] = 0;
			continue;
		}
		int64_t v = or_iexp_evaluate(z, base, q_c);
		if (!m_usable || v < 0 || v > mx) {
			ok = 0;
			exps[k] = 0;
			continue;
		}
		exps[k] = v;
		total += v;
	}
	int64_t denom = total > 1 ? total : 1;
	for (size_t k = 0; k < width; ++k) out_probs[k] = (exps[k] << 15) / denom;
	free(exps);
	return ok;
}

/* src/intmath.cpp:381-418 -- C28 core: round_away(b*r_a / 2^(q_b+62+e_a)) in 128 bits. */
int or_bias_reconcile_wide(int64_t b, int64_t q_b, int64_t r_a, int64_t e_a, int64_t* out) {
	s128 sum = (s128)q_b + 62 + (s128)e_a;
	if (sum < 0 || sum > 63) {
		*out = 0;
		return 0;
	}
	int exponent = (int)sum;
	s128 wide = (s128)b * (s128)r_a;
	uint64_t mask = exponent == 64 ? ~0ull : (((uint64_t)1 << exponent) - 1u);
	uint64_t rem = (uint64_t)wide & mask;
	uint64_t thr = (mask >> 1) + (wide < 0 ? 1u : 0u);
	s128 rounded = (wide >> exponent) + (rem > thr ? 1 : 0);
	*out = (int64_t)rounded;
	return rounded == (s128)(int64_t)rounded;
}

/* src/silu_lut.cpp:16-67 -- Q15 sigmoid by 1025-node table, Q12 sub-node interpolation. */
int32_t or_silu_sigmoid_q15(const int32_t* table, int8_t code, int64_t m, int e) {
	const int N = 1024, QIDX = 12, LOG2K = 5;
	int64_t term = (int64_t)code * m;
	int shift = e + LOG2K + QIDX;
	int64_t pos = shift >= 0 ? (term << shift) : or_rdbpot64(term, -shift);
	const int64_t hi_dom = (int64_t)N << QIDX;
	pos += hi_dom / 2;
	if (pos < 0) pos = 0;
	else if (pos > hi_dom) pos = hi_dom;
	int64_t i0 = pos >> QIDX;
	if (i0 > N - 1) i0 = N - 1;
	int64_t frac = pos - (i0 << QIDX);
	int64_t lo = table[i0], hi = table[i0 + 1];
	int64_t delta = or_rdbpot64(frac * (hi - lo), QIDX);
	return (int32_t)(lo + delta);
}

/* ================= funnel: src/forward/checked_chain_funnel.cpp ================= */

/* checked_chain_funnel.cpp:157-180 -- product of two carried scales, renormalized. */
or_scale or_combine_scale(or_scale a, or_scale b) {
	int64_t e = sat_add64(sat_add64(a.e, b.e), 31);
	int64_t m = or_srdhm((int32_t)a.m, (int32_t)b.m);
	if (m < ((int64_t)1 << 30)) {
		m <<= 1;
		e -= 1;
	}
	or_scale r = {m, e};
	return r;
}

static int fits_i32(int64_t m) { return m >= I32_MIN && m <= I32_MAX; }

/* checked_chain_funnel.cpp:257-364 -- max-abs, normalize, reciprocal, left-associated scale
 * fold (incoming..., site, D'-factor), per-element code. */
int or_requant_chain(const int64_t* row, size_t n, const or_scale* incoming, size_t n_in, or_scale site,
                     int8_t* out_codes, or_scale* out_scale) {
	for (size_t i = 0; i < n_in; ++i)
		if (!fits_i32(incoming[i].m)) return OR_CARRIED_SCALE_MANTISSA_OUT_OF_DOMAIN;
	if (!fits_i32(site.m)) return OR_CARRIED_SCALE_MANTISSA_OUT_OF_DOMAIN;
	int64_t dp = or_max_abs_wide(row, n);
	if (dp > ((int64_t)1 << 31)) return OR_CHAIN_INPUT_OUT_OF_DOMAIN;
	int s;
	int64_t dn = or_normalize_scale(dp, &s);
	int64_t r = or_reciprocal(dn);
	or_scale running = {0, 0};
	int have = 0, ok = 1;
	or_scale factors[8];
	size_t nf = 0;
	for (size_t i = 0; i < n_in; ++i) factors[nf++] = incoming[i];
	factors[nf++] = site;
	factors[nf].m = dn;
	factors[nf].e = -(int64_t)s;
	nf++;
	for (size_t i = 0; i < nf && ok; ++i) {
		running = have ? or_combine_scale(running, factors[i]) : factors[i];
		have = 1;
		ok = fits_i32(running.m);
	}
	if (!ok) return OR_CARRIED_SCALE_MANTISSA_OUT_OF_DOMAIN;
	for (size_t i = 0; i < n; ++i) out_codes[i] = or_requant_code_wide(row[i], r, s);
	*out_scale = running;
	return OR_OK;
}

/* checked_chain_funnel.cpp:520-583 */
int or_check_softmax_width(int64_t q_b, int64_t q_c, size_t width) {
	if (q_c < 0) return OR_SOFTMAX_ROW_WIDTH_OUT_OF_DOMAIN;
	if (width == 0) return OR_SOFTMAX_ROW_WIDTH_OUT_OF_DOMAIN;
	s128 m128 = (s128)q_b * q_b + (s128)q_c;
	if (m128 > (s128)I64_MAX || m128 > (s128)SOFTMAX_MAX_SAFE) return OR_SOFTMAX_ROW_WIDTH_OUT_OF_DOMAIN;
	int64_t m = (int64_t)m128;
	if (m != 0 && width > (size_t)(I64_MAX / m)) return OR_SOFTMAX_ROW_WIDTH_OUT_OF_DOMAIN;
	return OR_OK;
}

/* ================= sites: src/forward/forward_sites.cpp ================= */

/* forward_sites.cpp:461-470 -- identity passes through; else MBQM of the int32-truncated acc. */
int64_t or_apply_fold(int64_t acc, int32_t identity, int32_t mult, int32_t shift) {
	if (identity != 0) return acc;
	return (int64_t)or_mbqm((int32_t)acc, mult, shift);
}

/* forward_sites.cpp:472-481 */
int64_t or_apply_amp_fold(int64_t acc, int32_t identity, int32_t mult, int32_t exponent) {
	if (identity != 0) return acc;
	int32_t hi = or_srdhm((int32_t)acc, mult);
	if (exponent >= 0) return (int64_t)or_rdbpot32(hi, exponent);
	return (int64_t)or_sat_shl32(hi, -exponent);
}

static int64_t sat_sub64(int64_t a, int64_t b) {
	int64_t out = (int64_t)((uint64_t)a - (uint64_t)b);
	int ovf = ((a >= 0) != (b >= 0)) && ((out >= 0) != (a >= 0));
	if (!ovf) return out;
	return a >= 0 ? I64_MAX : I64_MIN;
}

/* forward_sites.cpp:389-395 */
static int64_t composed_exponent(int64_t e_a, int64_t e_t) {
	int64_t k = sat_sub64(62, sat_sub64(e_a, e_t));
	if (k > 4096) k = 4096;
	if (k < -4096) k = -4096;
	return k;
}

/* forward_sites.cpp:513-653 -- round_away(branch*m_a*r_t / 2^(62-(e_a-e_t))), exact left shift
 * for a negative exponent; counts clamps and reports an int64 overflow of the magnitude. */
int64_t or_landing_rescale(int64_t branch, int64_t m_a, int64_t r_t, int64_t e_a, int64_t e_t,
                           uint64_t* sat_count, int* exceeded_i64) {
	int neg = (branch < 0) != (m_a < 0);
	uint64_t ab = branch < 0 ? (~(uint64_t)branch + 1u) : (uint64_t)branch;
	uint64_t am = m_a < 0 ? (~(uint64_t)m_a + 1u) : (uint64_t)m_a;
	u128 mag = (u128)ab * am * (uint64_t)r_t; /* wraps mod 2^128 exactly like U128MulSmall */
	int64_t k = composed_exponent(e_a, e_t);
	int64_t raw;
	int exc_clamp, exc_i64;
	if (k >= 0) {
		u128 doubled = mag + mag;
		u128 one_k = k >= 128 ? 0 : ((u128)1 << k);
		u128 rounded = doubled + one_k;
		u128 q = (k + 1 >= 128) ? 0 : (rounded >> (k + 1));
		uint64_t qhi = (uint64_t)(q >> 64), qlo = (uint64_t)q;
		exc_clamp = (qhi != 0) || qlo > 127;
		exc_i64 = (qhi != 0) || qlo > (uint64_t)I64_MAX;
		raw = (int64_t)qlo;
	} else {
		int shift = (int)(-k);
		u128 shifted = shift >= 128 ? 0 : (mag << shift);
		if (shift >= 128) {
			exc_clamp = mag != 0;
			exc_i64 = exc_clamp;
		} else {
			u128 verify = shifted >> shift;
			int lost = verify != mag;
			uint64_t shi = (uint64_t)(shifted >> 64), slo = (uint64_t)shifted;
			exc_clamp = lost || shi != 0 || slo > 127;
			exc_i64 = lost || shi != 0 || slo > (uint64_t)I64_MAX;
		}
		raw = (int64_t)(uint64_t)shifted;
	}
	if (neg) raw = (int64_t)(0u - (uint64_t)raw);
	if (sat_count && (exc_clamp || raw < -127 || raw > 127)) *sat_count += 1;
	if (exceeded_i64) *exceeded_i64 = exc_i64;
	return raw;
}

/* forward_sites.cpp:655-661 */
static int64_t clamp_code(int64_t v) { return v > 127 ? 127 : (v < -127 ? -127 : v); }

/* forward_sites.cpp:399-408 */
static int64_t floor_div(int64_t a, int64_t b) {
	int64_t q = a / b, r = a % b;
	return (r != 0 && r < 0) ? q - 1 : q;
}

/* forward_sites.cpp:410-459 -- integer RMSNorm; the incoming scale is not folded. */
int or_rmsnorm_site(const int8_t* h, const int32_t* g, size_t n, or_scale site, int8_t* out,
                    or_scale* out_scale) {
	int64_t sumsq = 0;
	for (size_t i = 0; i < n; ++i) sumsq += (int64_t)h[i] * h[i];
	int64_t root = or_isqrt(floor_div(sumsq << 32, (int64_t)n));
	if (root < 1) root = 1;
	int64_t* wide = (int64_t*)malloc(n * sizeof(int64_t));
	for (size_t i = 0; i < n; ++i) wide[i] = floor_div((int64_t)h[i] << 32, root) * (int64_t)g[i];
	int st = or_requant_chain(wide, n, NULL, 0, site, out, out_scale);
	free(wide);
	return st;
}

/* forward_sites.cpp:763-787 */
int or_embed_entry(const or_model* m, int32_t token, int8_t* out, or_scale* out_scale) {
	if (token < 0 || token >= (int32_t)m->vocab) return OR_TOKEN_ID_OUT_OF_RANGE;
	const int8_t* row = m->embed + (size_t)token * m->hidden;
	int64_t* wide = (int64_t*)malloc(m->hidden * sizeof(int64_t));
	for (size_t i = 0; i < m->hidden; ++i) wide[i] = row[i];
	int st = or_requant_chain(wide, m->hidden, NULL, 0, m->embed_sc, out, out_scale);
	free(wide);
	return st;
}

/* checked_chain_funnel.cpp:402-405, 484-499 */
static int check_silu_scale(int64_t m, int64_t e) {
	const int64_t max_abs_m = ((int64_t)1 << 31) - 1;
	if (m < -max_abs_m || m > max_abs_m) return OR_SILU_COMPOSITION_SCALE_OUT_OF_DOMAIN;
	if (e < -80 || e > 8) return OR_SILU_COMPOSITION_SCALE_OUT_OF_DOMAIN;
	return OR_OK;
}

/* forward_sites.cpp:796-864 -- gate * sigmoidQ15(gate) * up, funnel with {gate, up}. */
int or_mlp_act_site(const int8_t* gate, or_scale gs, const int8_t* up, or_scale us, size_t n,
                    const int32_t* table, or_scale site, int8_t* out, or_scale* out_scale) {
	int st = check_silu_scale(gs.m, gs.e);
	if (st) return st;
	int64_t* wide = (int64_t*)malloc(n * sizeof(int64_t));
	for (size_t i = 0; i < n; ++i) {
		int32_t sig = or_silu_sigmoid_q15(table, gate[i], gs.m, (int)gs.e);
		wide[i] = (int64_t)gate[i] * sig * (int64_t)up[i];
	}
	or_scale inc[2] = {gs, us};
	st = or_requant_chain(wide, n, inc, 2, site, out, out_scale);
	free(wide);
	return st;
}

/* forward_sites.cpp:871-989 -- branch rescaled into the stream's scale, plus stream. */
int or_residual_site(const int8_t* branch, or_scale bs, const int8_t* stream, or_scale ss, size_t n,
                     or_scale site, int8_t* out, or_scale* out_scale) {
	if (!fits_i32(ss.m)) return OR_CARRIED_SCALE_MANTISSA_OUT_OF_DOMAIN;
	int64_t r_h = or_reciprocal(ss.m);
	int64_t* wide = (int64_t*)malloc(n * sizeof(int64_t));
	int bad = 0;
	for (size_t i = 0; i < n; ++i) {
		int exc = 0;
		int64_t rec = or_landing_rescale(branch[i], bs.m, r_h, bs.e, ss.e, NULL, &exc);
		if (exc) {
			bad = 1;
			continue;
		}
		wide[i] = rec + stream[i];
	}
	int st = OR_RESIDUAL_RECONCILIATION_MAGNITUDE_OUT_OF_DOMAIN;
	if (!bad) st = or_requant_chain(wide, n, &ss, 1, site, out, out_scale);
	free(wide);
	return st;
}

/* src/matmul.cpp:466-509 -- exact int64 dot of every activation row with every weight row. */
void or_gemm_i8(const int8_t* a, const int8_t* w, size_t m, size_t k, size_t n, int64_t* out) {
	for (size_t j = 0; j < n; ++j) {
		const int8_t* wr = w + j * k;
		for (size_t t = 0; t < m; ++t) {
			const int8_t* ar = a + t * k;
			int64_t acc = 0;
			for (size_t i = 0; i < k; ++i) acc += (int32_t)ar[i] * (int32_t)wr[i];
			out[t * n + j] = acc;
		}
	}
}

/* forward_sites.cpp:1051-1103 -- u = A x, amplifying fold, clamp, delta = B u, amplifying
 * fold, added into acc. */
static void lora_delta(const int8_t* x, size_t in_ch, const or_lora_proj* lp, uint32_t rank,
                       size_t out_ch, int64_t* acc) {
	if (!lp || !lp->a || !lp->b || !lp->u_fold || !lp->d_fold || rank == 0) return;
	int64_t* u_acc = (int64_t*)malloc(rank * sizeof(int64_t));
	int8_t* u8 = (int8_t*)malloc(rank);
	int64_t* d = (int64_t*)malloc(out_ch * sizeof(int64_t));
	or_gemm_i8(x, lp->a, 1, in_ch, rank, u_acc);
	for (uint32_t k = 0; k < rank; ++k) {
		const int32_t* f = lp->u_fold + 3 * k;
		u8[k] = (int8_t)clamp_code(or_apply_amp_fold(u_acc[k], f[0], f[1], f[2]));
	}
	or_gemm_i8(u8, lp->b, 1, rank, out_ch, d);
	for (size_t i = 0; i < out_ch; ++i) {
		const int32_t* f = lp->d_fold + 3 * i;
		acc[i] += or_apply_amp_fold(d[i], f[0], f[1], f[2]);
	}
	free(u_acc);
	free(u8);
	free(d);
}

/* forward_sites.cpp:1015-1036 -- two passes so a rejection leaves acc untouched. */
static int bias_row(int64_t* acc, size_t n, const int64_t* bias, or_scale in_scale) {
	s128 ex = (s128)30 + 62 + (s128)in_scale.e;
	if (ex < 0 || ex > 63) return OR_RDBPOT_EXPONENT_OUT_OF_DOMAIN;
	int64_t r_a = or_reciprocal(in_scale.m);
	for (size_t i = 0; i < n; ++i) {
		int64_t term;
		if (!or_bias_reconcile_wide(bias[i], 30, r_a, in_scale.e, &term))
			return OR_BIAS_RECONCILE_PRODUCT_OUT_OF_DOMAIN;
		uint64_t s = (uint64_t)acc[i] + (uint64_t)term;
		if (((((uint64_t)acc[i] ^ (uint64_t)term) >> 63) == 0) && ((((uint64_t)acc[i] ^ s) >> 63) != 0))
			return OR_BIAS_RECONCILE_PRODUCT_OUT_OF_DOMAIN;
	}
	for (size_t i = 0; i < n; ++i) {
		int64_t term;
		or_bias_reconcile_wide(bias[i], 30, r_a, in_scale.e, &term);
		acc[i] += term;
	}
	return OR_OK;
}

/* forward_sites.cpp:1114-1146 (FunnelProjectedRow), acc filled by the caller. */
static int funnel_projected_row(int64_t* acc, const int8_t* x, or_scale in_scale, size_t in_ch,
                                size_t out_ch, const int32_t* fold, const int64_t* bias,
                                const or_lora_proj* lora, uint32_t rank, or_scale site, int8_t* out,
                                or_scale* out_scale) {
	for (size_t i = 0; i < out_ch; ++i) acc[i] = or_apply_fold(acc[i], fold[3 * i], fold[3 * i + 1], fold[3 * i + 2]);
	lora_delta(x, in_ch, lora, rank, out_ch, acc);
	if (bias) {
		int st = bias_row(acc, out_ch, bias, in_scale);
		if (st) return st;
	}
	return or_requant_chain(acc, out_ch, &in_scale, 1, site, out, out_scale);
}

int or_project_row(const int8_t* x, or_scale in_scale, size_t in_ch, size_t out_ch, const int8_t* w,
                   const int32_t* fold, const int64_t* bias, const or_lora_proj* lora, uint32_t rank,
                   or_scale site, int8_t* out, or_scale* out_scale) {
	int64_t* acc = (int64_t*)malloc(out_ch * sizeof(int64_t));
	or_gemm_i8(x, w, 1, in_ch, out_ch, acc);
	int st = funnel_projected_row(acc, x, in_scale, in_ch, out_ch, fold, bias, lora, rank, site, out,
	                              out_scale);
	free(acc);
	return st;
}

/* ---------------- KV layout: forward_sites.cpp:1227-1269 ---------------- */
size_t or_kv_block_bytes(const or_model* m) {
	return (size_t)m->layers * (size_t)m->context_cap * m->kv_heads * m->head_dim * 2;
}

static int8_t* key_row(const or_model* m, int8_t* kv, uint32_t l, size_t kvh, int64_t pos) {
	size_t half = (size_t)m->context_cap * m->kv_heads * m->head_dim;
	return kv + (size_t)l * half * 2 + kvh * (size_t)m->context_cap * m->head_dim + (size_t)pos * m->head_dim;
}

static int8_t* value_row(const or_model* m, int8_t* kv, uint32_t l, size_t kvh, int64_t pos) {
	size_t half = (size_t)m->context_cap * m->kv_heads * m->head_dim;
	return key_row(m, kv, l, kvh, pos) + half;
}

/* forward_sites.cpp:663-761 (ROP1 row read: forward_sites.cpp:48-53) */
static int rope_site(const or_model* m, const int8_t* row, int64_t pos, int8_t* out) {
	if (pos < 0 || pos >= m->context_cap) return OR_POSITION_OVER_CAP;
	size_t pairs = m->head_dim / 2;
	for (size_t i = 0; i < pairs; ++i) {
		int32_t c = (int32_t)m->rope_cos[(size_t)pos * pairs + i];
		int32_t s = (int32_t)m->rope_sin[(size_t)pos * pairs + i];
		int64_t xr, yr;
		or_rope_pair(row[2 * i], row[2 * i + 1], c, s, &xr, &yr);
		out[2 * i] = (int8_t)clamp_code(xr);
		out[2 * i + 1] = (int8_t)clamp_code(yr);
	}
	return OR_OK;
}

/* forward_sites.cpp:1281-1418 (LandTokenKVRow, Option G off). */
static int land_kv(const or_model* m, const or_layer* lw, uint32_t l, int64_t* kacc, int64_t* vacc,
                   const int8_t* normed, or_scale ns, int64_t pos, int8_t* kv, uint64_t* sat) {
	size_t kvh = (size_t)m->kv_heads * m->head_dim;
	for (size_t i = 0; i < kvh; ++i) {
		const int32_t* fk = lw->fold[OR_K] + 3 * i;
		const int32_t* fv = lw->fold[OR_V] + 3 * i;
		kacc[i] = or_apply_fold(kacc[i], fk[0], fk[1], fk[2]);
		vacc[i] = or_apply_fold(vacc[i], fv[0], fv[1], fv[2]);
	}
	lora_delta(normed, m->hidden, lw->lora[OR_K], lw->lora_rank, kvh, kacc);
	lora_delta(normed, m->hidden, lw->lora[OR_V], lw->lora_rank, kvh, vacc);
	if (lw->bias[1]) {
		int st = bias_row(kacc, kvh, lw->bias[1], ns);
		if (st) return st;
	}
	if (lw->bias[2]) {
		int st = bias_row(vacc, kvh, lw->bias[2], ns);
		if (st) return st;
	}
	for (size_t h = 0; h < m->kv_heads; ++h) {
		int8_t* kr = key_row(m, kv, l, h, pos);
		int8_t* vr = value_row(m, kv, l, h, pos);
		for (size_t d = 0; d < m->head_dim; ++d) {
			size_t i = h * m->head_dim + d;
			kr[d] = (int8_t)clamp_code(
			    or_landing_rescale(kacc[i], ns.m, lw->kv_r_t_k[h], ns.e, lw->kv_e_t_k[h], sat, NULL));
		}
		for (size_t d = 0; d < m->head_dim; ++d) {
			size_t i = h * m->head_dim + d;
			vr[d] = (int8_t)clamp_code(
			    or_landing_rescale(vacc[i], ns.m, lw->kv_r_t_v[h], ns.e, lw->kv_e_t_v[h], sat, NULL));
		}
	}
	return OR_OK;
}

/* forward_sites.cpp:1748-1787 -- q rotated per head; the landed K row at `pos` rotated once per
 * kv head and written back. */
static int rope_q_and_k(const or_model* m, uint32_t l, const int8_t* q_codes, int64_t pos, int8_t* kv,
                        int8_t* q_rot) {
	size_t D = m->head_dim;
	size_t group = m->heads / m->kv_heads;
	int8_t* k_rot = (int8_t*)malloc((size_t)m->kv_heads * D);
	for (size_t h = 0; h < m->heads; ++h) {
		int st = rope_site(m, q_codes + h * D, pos, q_rot + h * D);
		if (st) {
			free(k_rot);
			return st;
		}
		size_t kvh = h / group;
		st = rope_site(m, key_row(m, kv, l, kvh, pos), pos, k_rot + kvh * D);
		if (st) {
			free(k_rot);
			return st;
		}
	}
	for (size_t kvh = 0; kvh < m->kv_heads; ++kvh) memcpy(key_row(m, kv, l, kvh, pos), k_rot + kvh * D, D);
	free(k_rot);
	return OR_OK;
}

/* forward_sites.cpp:1791-1905 -- per kv head: combine q scale with softmax_khead, derive the
 * i-exp triple, gate the width, score, softmax, PV, per-head ctx fold; one funnel over H. */
static int attention(const or_model* m, const or_layer* lw, uint32_t l, const int8_t* q_rot,
                     or_scale q_scale, int64_t pos, int8_t* kv, int8_t* ctx_codes, or_scale* ctx_scale) {
	size_t D = m->head_dim, H = m->hidden;
	size_t group = m->heads / m->kv_heads;
	size_t width = (size_t)pos + 1;
	int64_t ln2_q, b_q, ca_q;
	or_iexp_pinned(&ln2_q, &b_q, &ca_q);
	int64_t* ctx_wide = (int64_t*)malloc(H * sizeof(int64_t));
	int64_t* scores = (int64_t*)malloc(width * sizeof(int64_t));
	int64_t* probs = (int64_t*)malloc(width * sizeof(int64_t));
	int64_t tq_ln2[64], tq_b[64], tq_c[64];
	int derived[64] = {0};
	int st = OR_OK;
	for (size_t h = 0; h < m->heads && !st; ++h) {
		size_t kvh = h / group;
		if (!derived[kvh]) {
			int64_t km = lw->khead_m[kvh], ke = lw->khead_e[kvh];
			if (!fits_i32(q_scale.m) || !fits_i32(km)) {
				st = OR_CARRIED_SCALE_MANTISSA_OUT_OF_DOMAIN;
				break;
			}
			or_scale kh = {km, ke};
			or_scale sm = or_combine_scale(q_scale, kh);
			if (!fits_i32(sm.m)) {
				st = OR_CARRIED_SCALE_MANTISSA_OUT_OF_DOMAIN;
				break;
			}
			if (or_iexp_scale_constants(sm.m, sm.e, ln2_q, 30, b_q, 30, ca_q, 30, &tq_ln2[kvh], &tq_b[kvh],
			                            &tq_c[kvh]) != 0) {
				st = OR_IEXP_SCALE_DERIVATION_OUT_OF_DOMAIN;
				break;
			}
			derived[kvh] = 1;
		}
		st = or_check_softmax_width(tq_b[kvh], tq_c[kvh], width);
		if (st) break;
		const int8_t* qh = q_rot + h * D;
		for (size_t p = 0; p < width; ++p) {
			const int8_t* kr = key_row(m, kv, l, kvh, (int64_t)p);
			int64_t acc = 0;
			for (size_t d = 0; d < D; ++d) acc += (int32_t)qh[d] * (int32_t)kr[d];
			scores[p] = acc;
		}
		if (!or_softmax_row_q15(scores, width, tq_ln2[kvh], tq_b[kvh], tq_c[kvh], probs)) {
			st = OR_SOFTMAX_KERNEL_REFUSED_AFTER_GATE_ACCEPTED;
			break;
		}
		const int32_t* cf = lw->ctx_fold + 3 * h;
		for (size_t d = 0; d < D; ++d) {
			int64_t acc = 0;
			for (size_t p = 0; p < width; ++p) acc += probs[p] * (int64_t)value_row(m, kv, l, kvh, (int64_t)p)[d];
			ctx_wide[h * D + d] = or_apply_fold(acc, cf[0], cf[1], cf[2]);
		}
	}
	if (!st) st = or_requant_chain(ctx_wide, H, NULL, 0, lw->ctx_sc, ctx_codes, ctx_scale);
	free(ctx_wide);
	free(scores);
	free(probs);
	return st;
}

static int check_geometry(const or_model* m) {
	if (m->context_cap < 1) return OR_INVALID_CONTEXT_CAP;
	size_t nh = m->head_dim == 0 ? 0 : m->hidden / m->head_dim;
	if (nh == 0 || nh * m->head_dim != m->hidden) return OR_HEAD_DIM_GEOMETRY_MISMATCH;
	if (m->kv_heads == 0 || m->kv_heads > nh || nh % m->kv_heads != 0) return OR_KV_HEAD_GEOMETRY_MISMATCH;
	if (m->kv_heads > 64) return OR_KV_HEAD_GEOMETRY_MISMATCH; /* oracle table limit */
	return OR_OK;
}

/* forward_sites.cpp:1429-2014 -- sliced decode: up to `layer_budget` layers, one commit per
 * layer, context_length advanced after the last layer. */
static or_trace_fn g_trace_fn;
static void* g_trace_user;
void or_set_trace(or_trace_fn fn, void* user) {
	g_trace_fn = fn;
	g_trace_user = fn ? user : NULL;
}
static void trace_site(uint32_t layer, int site, const int8_t* codes, size_t n, or_scale sc) {
	if (g_trace_fn) g_trace_fn(g_trace_user, layer, site, codes, n, sc.m, sc.e);
}

int or_run_layer_loop(const or_model* m, or_seq* seq, uint32_t layer_budget, int8_t* kv) {
	if (layer_budget == 0) return OR_INVALID_LAYER_BUDGET;
	int st = check_geometry(m);
	if (st) return st;
	if (!seq->hidden) return OR_INVALID_HIDDEN_CODES;
	if (seq->layer_index >= m->layers) return OR_SEQUENCE_ALREADY_COMPLETE;
	if (seq->context_length < 0) return OR_POSITION_OVER_CAP;
	if (seq->context_length >= m->context_cap) return OR_KV_CAPACITY_EXHAUSTED;
	size_t H = m->hidden, I = m->inter, KVH = (size_t)m->kv_heads * m->head_dim;
	int64_t pos = seq->context_length;
	int8_t* normed = (int8_t*)malloc(H);
	int8_t* q = (int8_t*)malloc(H);
	int8_t* q_rot = (int8_t*)malloc(H);
	int8_t* ctx = (int8_t*)malloc(H);
	int8_t* o = (int8_t*)malloc(H);
	int8_t* attn_stream = (int8_t*)malloc(H);
	int8_t* gate = (int8_t*)malloc(I);
	int8_t* up = (int8_t*)malloc(I);
	int8_t* act = (int8_t*)malloc(I);
	int8_t* down = (int8_t*)malloc(H);
	int8_t* next = (int8_t*)malloc(H);
	int64_t* kacc = (int64_t*)malloc(KVH * sizeof(int64_t));
	int64_t* vacc = (int64_t*)malloc(KVH * sizeof(int64_t));
	uint32_t advanced = 0;
	while (advanced < layer_budget && seq->layer_index < m->layers) {
		uint32_t l = seq->layer_index;
		const or_layer* lw = &m->layer[l];
		or_scale ns, qs, cs, os, as, mns, gs, us, acts, ds, ss;
		uint32_t r = lw->lora_rank;
		if ((st = or_rmsnorm_site(seq->hidden, lw->attn_gain, H, lw->attn_norm_sc, normed, &ns))) break;
		trace_site(l, OR_SITE_ATTN_NORM, normed, H, ns);
		if ((st = or_project_row(normed, ns, H, H, lw->w[OR_Q], lw->fold[OR_Q], lw->bias[0], lw->lora[OR_Q],
		                         r, lw->q_sc, q, &qs)))
			break;
		trace_site(l, OR_SITE_Q, q, H, qs);
		or_gemm_i8(normed, lw->w[OR_K], 1, H, KVH, kacc);
		or_gemm_i8(normed, lw->w[OR_V], 1, H, KVH, vacc);
		if ((st = land_kv(m, lw, l, kacc, vacc, normed, ns, pos, kv, &seq->kv_saturation_count))) break;
		if ((st = rope_q_and_k(m, l, q, pos, kv, q_rot))) break;
		trace_site(l, OR_SITE_Q_ROT, q_rot, H, qs);
		if ((st = attention(m, lw, l, q_rot, qs, pos, kv, ctx, &cs))) break;
		trace_site(l, OR_SITE_CTX, ctx, H, cs);
		if ((st = or_project_row(ctx, cs, H, H, lw->w[OR_O], lw->fold[OR_O], NULL, lw->lora[OR_O], r, lw->o_sc, o,
		                         &os)))
			break;
		trace_site(l, OR_SITE_O, o, H, os);
		if ((st = or_residual_site(o, os, seq->hidden, seq->scale, H, lw->attn_res_sc, attn_stream, &as))) break;
		trace_site(l, OR_SITE_ATTN_RESIDUAL, attn_stream, H, as);
		if ((st = or_rmsnorm_site(attn_stream, lw->mlp_gain, H, lw->mlp_norm_sc, normed, &mns))) break;
		trace_site(l, OR_SITE_MLP_NORM, normed, H, mns);
		if ((st = or_project_row(normed, mns, H, I, lw->w[OR_GATE], lw->fold[OR_GATE], NULL, lw->lora[OR_GATE], r,
		                         lw->gate_sc, gate, &gs)))
			break;
		if ((st = or_project_row(normed, mns, H, I, lw->w[OR_UP], lw->fold[OR_UP], NULL, lw->lora[OR_UP], r,
		                         lw->up_sc, up, &us)))
			break;
		trace_site(l, OR_SITE_GATE, gate, I, gs);
		trace_site(l, OR_SITE_UP, up, I, us);
		if ((st = or_mlp_act_site(gate, gs, up, us, I, m->silu_table, lw->act_sc, act, &acts))) break;
		trace_site(l, OR_SITE_ACT, act, I, acts);
		if ((st = or_project_row(act, acts, I, H, lw->w[OR_DOWN], lw->fold[OR_DOWN], NULL, lw->lora[OR_DOWN], r,
		                         lw->down_sc, down, &ds)))
			break;
		trace_site(l, OR_SITE_DOWN, down, H, ds);
		if ((st = or_residual_site(down, ds, attn_stream, as, H, lw->mlp_res_sc, next, &ss))) break;
		trace_site(l, OR_SITE_MLP_RESIDUAL, next, H, ss);
		memcpy(seq->hidden, next, H);
		seq->scale = ss;
		seq->layer_index = l + 1;
		if (seq->layer_index == m->layers) seq->context_length += 1;
		++advanced;
	}
	free(normed); free(q); free(q_rot); free(ctx); free(o); free(attn_stream);
	free(gate); free(up); free(act); free(down); free(next); free(kacc); free(vacc);
	return st;
}

/* forward_sites.cpp:2098-2401 -- chunked prefill over the whole depth.  Every per-row step is
 * the same function the decode loop runs, in position order; the GEMMs are batched. */
int or_run_chunk(const or_model* m, int8_t* hid, or_scale* scales, size_t T, int64_t ctx_start, int8_t* kv,
                 uint64_t* sat) {
	if (T == 0) return OR_INVALID_LAYER_BUDGET;
	int st = check_geometry(m);
	if (st) return st;
	if (!hid || !scales) return OR_INVALID_HIDDEN_CODES;
	if (ctx_start < 0) return OR_POSITION_OVER_CAP;
	if (ctx_start > m->context_cap - (int64_t)T) return OR_KV_CAPACITY_EXHAUSTED;
	size_t H = m->hidden, I = m->inter, KVH = (size_t)m->kv_heads * m->head_dim;
	int8_t* normed = (int8_t*)malloc(T * H);
	int8_t* q = (int8_t*)malloc(T * H);
	int8_t* ctx = (int8_t*)malloc(T * H);
	int8_t* o = (int8_t*)malloc(T * H);
	int8_t* as_c = (int8_t*)malloc(T * H);
	int8_t* mn = (int8_t*)malloc(T * H);
	int8_t* gate = (int8_t*)malloc(T * I);
	int8_t* up = (int8_t*)malloc(T * I);
	int8_t* act = (int8_t*)malloc(T * I);
	int8_t* down = (int8_t*)malloc(T * H);
	int8_t* next = (int8_t*)malloc(T * H);
	int8_t* q_rot = (int8_t*)malloc(H);
	size_t maxn = I > H ? I : H;
	int64_t* acc = (int64_t*)malloc(T * maxn * sizeof(int64_t));
	int64_t* kacc = (int64_t*)malloc(T * KVH * sizeof(int64_t));
	int64_t* vacc = (int64_t*)malloc(T * KVH * sizeof(int64_t));
	or_scale* ns = (or_scale*)malloc(T * sizeof(or_scale) * 11);
	or_scale *qs = ns + T, *cs = ns + 2 * T, *os = ns + 3 * T, *ass = ns + 4 * T, *mns = ns + 5 * T;
	or_scale *gs = ns + 6 * T, *us = ns + 7 * T, *acts = ns + 8 * T, *ds = ns + 9 * T, *ss = ns + 10 * T;

#define BATCHED(XIN, XSC, KIN, NOUT, P, BIAS, SITE, OUT, OSC)                                            \
	do {                                                                                                 \
		or_gemm_i8(XIN, lw->w[P], T, KIN, NOUT, acc);                                                    \
		for (size_t t = 0; t < T && !st; ++t)                                                            \
			st = funnel_projected_row(acc + t * (NOUT), (XIN) + t * (KIN), (XSC)[t], KIN, NOUT, lw->fold[P], \
			                          BIAS, lw->lora[P], lw->lora_rank, SITE, (OUT) + t * (NOUT), &(OSC)[t]); \
	} while (0)

/* every token's row of one site, in position order */
#define TRACE_ROWS(SITE, CODES, N, SC)                                                \
	do {                                                                              \
		for (size_t t = 0; t < T && !st; ++t) trace_site(l, SITE, (CODES) + t * (N), N, (SC)[t]); \
	} while (0)

	for (uint32_t l = 0; l < m->layers && !st; ++l) {
		const or_layer* lw = &m->layer[l];
		for (size_t t = 0; t < T && !st; ++t)
			st = or_rmsnorm_site(hid + t * H, lw->attn_gain, H, lw->attn_norm_sc, normed + t * H, &ns[t]);
		if (st) break;
		TRACE_ROWS(OR_SITE_ATTN_NORM, normed, H, ns);
		BATCHED(normed, ns, H, H, OR_Q, lw->bias[0], lw->q_sc, q, qs);
		if (st) break;
		TRACE_ROWS(OR_SITE_Q, q, H, qs);
		or_gemm_i8(normed, lw->w[OR_K], T, H, KVH, kacc);
		or_gemm_i8(normed, lw->w[OR_V], T, H, KVH, vacc);
		for (size_t t = 0; t < T && !st; ++t) {
			int64_t pos = ctx_start + (int64_t)t;
			st = land_kv(m, lw, l, kacc + t * KVH, vacc + t * KVH, normed + t * H, ns[t], pos, kv, sat);
			if (!st) st = rope_q_and_k(m, l, q + t * H, pos, kv, q_rot);
			if (!st) trace_site(l, OR_SITE_Q_ROT, q_rot, H, qs[t]);
			if (!st) st = attention(m, lw, l, q_rot, qs[t], pos, kv, ctx + t * H, &cs[t]);
		}
		if (st) break;
		TRACE_ROWS(OR_SITE_CTX, ctx, H, cs);
		BATCHED(ctx, cs, H, H, OR_O, NULL, lw->o_sc, o, os);
		if (st) break;
		TRACE_ROWS(OR_SITE_O, o, H, os);
		for (size_t t = 0; t < T && !st; ++t)
			st = or_residual_site(o + t * H, os[t], hid + t * H, scales[t], H, lw->attn_res_sc, as_c + t * H, &ass[t]);
		if (st) break;
		TRACE_ROWS(OR_SITE_ATTN_RESIDUAL, as_c, H, ass);
		for (size_t t = 0; t < T && !st; ++t)
			st = or_rmsnorm_site(as_c + t * H, lw->mlp_gain, H, lw->mlp_norm_sc, mn + t * H, &mns[t]);
		if (st) break;
		TRACE_ROWS(OR_SITE_MLP_NORM, mn, H, mns);
		BATCHED(mn, mns, H, I, OR_GATE, NULL, lw->gate_sc, gate, gs);
		if (st) break;
		BATCHED(mn, mns, H, I, OR_UP, NULL, lw->up_sc, up, us);
		if (st) break;
		TRACE_ROWS(OR_SITE_GATE, gate, I, gs);
		TRACE_ROWS(OR_SITE_UP, up, I, us);
		for (size_t t = 0; t < T && !st; ++t)
			st = or_mlp_act_site(gate + t * I, gs[t], up + t * I, us[t], I, m->silu_table, lw->act_sc, act + t * I,
			                     &acts[t]);
		if (st) break;
		TRACE_ROWS(OR_SITE_ACT, act, I, acts);
		BATCHED(act, acts, I, H, OR_DOWN, NULL, lw->down_sc, down, ds);
		if (st) break;
		TRACE_ROWS(OR_SITE_DOWN, down, H, ds);
		for (size_t t = 0; t < T && !st; ++t)
			st = or_residual_site(down + t * H, ds[t], as_c + t * H, ass[t], H, lw->mlp_res_sc, next + t * H, &ss[t]);
		if (st) break;
		TRACE_ROWS(OR_SITE_MLP_RESIDUAL, next, H, ss);
		memcpy(hid, next, T * H);
		memcpy(scales, ss, T * sizeof(or_scale));
	}
#undef TRACE_ROWS
#undef BATCHED
	free(normed); free(q); free(ctx); free(o); free(as_c); free(mn); free(gate); free(up); free(act);
	free(down); free(next); free(q_rot); free(acc); free(kacc); free(vacc); free(ns);
	return st;
}

/* src/sslm_abi.cpp:2280-2289 + forward_sites.cpp:2412-2417 + checked_chain_funnel.cpp:366-384:
 * final RMSNorm, LM-head GEMV, checked int32 narrowing. */
int or_final_logits(const or_model* m, const int8_t* hidden, int32_t* out_logits) {
	size_t H = m->hidden;
	int8_t* fc = (int8_t*)malloc(H);
	or_scale fs;
	int st = or_rmsnorm_site(hidden, m->final_gain, H, m->final_sc, fc, &fs);
	if (!st) {
		int64_t* wide = (int64_t*)malloc((size_t)m->vocab * sizeof(int64_t));
		or_gemm_i8(fc, m->head, 1, H, m->vocab, wide);
		for (size_t i = 0; i < m->vocab && !st; ++i)
			if (wide[i] > I32_MAX || wide[i] < I32_MIN) st = OR_LOGIT_NARROWING_OVERFLOW;
		if (!st)
			for (size_t i = 0; i < m->vocab; ++i) out_logits[i] = (int32_t)wide[i];
		free(wide);
	}
	free(fc);
	return st;
}

/* forward_sites.cpp:2427-2437 -- lowest index wins ties. */
int32_t or_argmax(const int32_t* logits, size_t n) {
	int32_t best = 0, bv = logits[0];
	for (size_t i = 1; i < n; ++i)
		if (logits[i] > bv) {
			bv = logits[i];
			best = (int32_t)i;
		}
	return best;
}
