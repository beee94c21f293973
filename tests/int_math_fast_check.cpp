// Host check of the exact fast forms in int_math.h (iexp_fast, div_rcp) against the forms they
// replace (iexp_element, div_floor_pos): random and edge-case inputs; prints the mismatch counts.
#include "int_math.h"
#include <cstdlib>
#include <cstdio>
#include <random>
using namespace sslm;
int main(int argc, char** argv) {
	const int N = argc > 1 ? atoi(argv[1]) : 4000000;
	std::mt19937_64 rng(1);
	long bad = 0, n = 0, nonneg = 0;
	for (int it = 0; it < N; ++it) {
		int64_t qln2 = 1 + (int64_t)(rng() % (it % 3 == 0 ? 1000ull : (it % 3 == 1 ? (1ull << 30) : (1ull << 58) / 30)));
		if (it % 101 == 0) qln2 = kI64Max / 30 + (int64_t)(rng() % 3) - 1;
		int64_t qb = (int64_t)(rng() % (1ull << 23)) - (1ll << 22);
		int64_t qc = (int64_t)(rng() % (1ull << 46));
		if (it % 7 == 0) qb = (int64_t)(rng() % 65536);
		if ((s128)qb * qb + qc > kSoftmaxMaxSafe) continue;
		int64_t cm = softmax_ceiling(qb, qc);
		int64_t sh = -(int64_t)(rng() % (uint64_t)(it % 2 ? 40 * (uint64_t)(qln2 > (1ll << 40) ? (1ll << 40) : qln2) + 1 : 4294967296ull));
		if (it % 5 == 0) sh = -(int64_t)(rng() % 64);
		int64_t a = iexp_element(sh, qln2, qb, qc, cm);
		int64_t b = iexp_fast(sh, qln2, 1.0 / (double)qln2, qb, qc, cm);
		++n;
		nonneg += a >= 0;
		if (a != b) { if (bad < 10) printf("iexp mismatch sh=%lld qln2=%lld qb=%lld qc=%lld: %lld vs %lld\n", (long long)sh, (long long)qln2, (long long)qb, (long long)qc, (long long)a, (long long)b); ++bad; }
	}
	printf("iexp: %ld cases (%ld accepted), %ld mismatches\n", n, nonneg, bad);
	// the 32-bit form on its whole admitted domain: q_ln2 up to (2^31 - 1) / 30, |q_b| + q_ln2 up
	// to 2^31 - 1 (edges included), shifts at and around multiples of q_ln2 and past 30 q_ln2
	long bs = 0, ns = 0, acc_s = 0;
	for (int it = 0; it < N; ++it) {
		int64_t qln2 = 1 + (int64_t)(rng() % (it % 3 == 0 ? 1000ull : (uint64_t)(kI32Max / 30)));
		if (it % 53 == 0) qln2 = kI32Max / 30 - (int64_t)(rng() % 2);
		const int64_t room = kI32Max - qln2;
		int64_t qb = (int64_t)(rng() % (uint64_t)(2 * (it % 4 ? (room < (1ll << 23) ? room : (1ll << 23)) : room) + 1)) -
		             (it % 4 ? (room < (1ll << 23) ? room : (1ll << 23)) : room);
		if (it % 59 == 0) qb = (it & 1) ? room : -room;
		int64_t qc = (int64_t)(rng() % (1ull << 46));
		if ((s128)qb * qb + qc > kSoftmaxMaxSafe) qc = 0;
		if ((s128)qb * qb + qc > kSoftmaxMaxSafe) continue;
		const int64_t cm = softmax_ceiling(qb, qc);
		if (!iexp_small_ok(qln2, qb, cm)) continue;
		int64_t sh;
		const int kind = it % 4;
		if (kind == 0) sh = -(int64_t)(rng() % (31 * (uint64_t)qln2 + 1));
		else if (kind == 1) sh = -((int64_t)(rng() % 31) * qln2 + (int64_t)(rng() % 3) - 1);
		else if (kind == 2) sh = -(int64_t)(rng() % (1ull << 33));
		else sh = -(int64_t)(rng() % 64);
		if (sh > 0) sh = 0;
		const int64_t a = iexp_element(sh, qln2, qb, qc, cm);
		const int64_t b = iexp_small(sh, (int32_t)qln2, 1.0 / (double)qln2, (int32_t)qb, qc, cm);
		++ns;
		acc_s += a >= 0;
		if (a != b) {
			if (bs < 10) printf("iexp_small mismatch sh=%lld qln2=%lld qb=%lld qc=%lld: %lld vs %lld\n", (long long)sh, (long long)qln2, (long long)qb, (long long)qc, (long long)a, (long long)b);
			++bs;
		}
	}
	printf("iexp_small: %ld cases (%ld accepted), %ld mismatches\n", ns, acc_s, bs);
	long bd = 0;
	for (int it = 0; it < N; ++it) {
		int64_t d = 1 + (int64_t)(rng() % (it % 2 ? (1ull << 60) : 100000ull));
		int64_t e = (int64_t)(rng() % (uint64_t)(d < (1ll << 47) ? d + 1 : (1ll << 47)));
		if (it % 3 == 0) e = d < (1ll << 47) ? d : e;
		int64_t q1 = div_floor_pos(e << 15, d), q2 = div_rcp(e << 15, d, 1.0 / (double)d, 32768);
		if (q1 != q2) { if (bd < 10) printf("div mismatch %lld/%lld: %lld vs %lld\n", (long long)e, (long long)d, (long long)q1, (long long)q2); ++bd; }
	}
	printf("div: %ld mismatches\n", bd);
	long bq = 0;
	for (int it = 0; it < N; ++it) {
		int64_t d = 1 + (int64_t)(rng() % (it % 2 ? (1ull << 38) - 1 : 100000ull));
		if (it % 97 == 0) d = (1ll << 38) - 1 - (int64_t)(rng() % 4);
		int64_t e = (int64_t)(rng() % (uint64_t)(d + 1));
		if (it % 3 == 0) e = d;
		if (it % 5 == 0) {  // e just around a multiple of d / 2^15
			const int64_t k = (int64_t)(rng() % 32769);
			e = (k * d) >> 15;
			e += (int64_t)(rng() % 3) - 1;
			e = e < 0 ? 0 : (e > d ? d : e);
		}
		if (!div_q15_small_ok(d)) continue;
		const int64_t q1 = div_floor_pos(e << 15, d);
		const int32_t q2 = div_q15_small(e, (double)d, 1.0 / (double)d);
		if (q1 != q2) { if (bq < 10) printf("div_q15_small mismatch %lld/%lld: %lld vs %d\n", (long long)e, (long long)d, (long long)q1, q2); ++bq; }
	}
	printf("div_q15_small: %ld mismatches\n", bq);
	// the RMSNorm per-code quotient: every code against the table form, every root up to 2^16
	// and random roots up to 2^24 (the norm's roots stay below 2^23)
	long bn = 0, nn = 0;
	auto fd_table = [](int64_t v, int64_t root) {
		const int64_t x = v << 32;
		return x >= 0 ? div_floor_pos(x, root) : -div_floor_pos(-x + root - 1, root);
	};
	for (int64_t it = 0; it < (1 << 16) + N / 8; ++it) {
		int64_t root = it < (1 << 16) ? 1 + it : 1 + (int64_t)(rng() % (1ull << 24));
		if (it % 1009 == 0) root = (1ll << 24) - 1 - (int64_t)(rng() % 4);
		const double rd = (double)root, inv = 1.0 / rd;
		for (int v = -128; v < 128; ++v) {
			++nn;
			const int64_t a = fd_table(v, root), b = norm_fd(v, rd, inv);
			if (a != b) { if (bn < 10) printf("norm_fd mismatch v=%d root=%lld: %lld vs %lld\n", v, (long long)root, (long long)a, (long long)b); ++bn; }
		}
	}
	printf("norm_fd: %ld cases, %ld mismatches\n", nn, bn);
}
