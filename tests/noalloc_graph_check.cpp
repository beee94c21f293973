// sslm_hip_gemm_requant_noalloc on a created stream and inside HIP graph capture (the callers it is
// for): one captured call, replayed three times with new inputs written into the same buffers and
// eager work (the allocating entry point, synchronous copies) between replays; every replay must
// equal sslm_hip_gemm_requant on the same inputs bit for bit.  Prints "ok" on success.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#include <vector>

#include "../include/sslm_hip.h"

#define CK(x)                                                                          \
	do {                                                                               \
		hipError_t e_ = (x);                                                           \
		if (e_ != hipSuccess) {                                                        \
			printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);      \
			return 1;                                                                  \
		}                                                                              \
	} while (0)

static uint32_t g_s = 12345;
static int8_t rnd8() {
	g_s = g_s * 1664525u + 1013904223u;
	return (int8_t)((int)((g_s >> 24) % 255) - 127);
}

int main() {
	const int m = 32, k = 896, n = 4864;
	const int64_t in_m = 1 << 30, in_e = -37, site_m = 1518500250, site_e = -45;  // configuration 0's scales
	int8_t *a, *w, *codes, *codes_ref;
	int32_t *fold, *st, *st_ref;
	int64_t *me, *me_ref;
	CK(hipMalloc(&a, (size_t)m * k));
	CK(hipMalloc(&w, (size_t)n * k));
	CK(hipMalloc(&fold, (size_t)n * 12));
	CK(hipMalloc(&codes, (size_t)m * n));
	CK(hipMalloc(&codes_ref, (size_t)m * n));
	CK(hipMalloc(&st, m * 4));
	CK(hipMalloc(&st_ref, m * 4));
	CK(hipMalloc(&me, m * 16));
	CK(hipMalloc(&me_ref, m * 16));
	std::vector<int32_t> hf((size_t)n * 3);
	for (int j = 0; j < n; ++j) {
		hf[3 * j] = 0;
		g_s = g_s * 1664525u + 1013904223u;
		hf[3 * j + 1] = (int32_t)((1u << 30) + (g_s >> 2) % (1u << 30));
		hf[3 * j + 2] = 8 + (int)(g_s % 13);  // multiplier in [2^30, 2^31), shift in [8, 20]
	}
	CK(hipMemcpy(fold, hf.data(), hf.size() * 4, hipMemcpyHostToDevice));
	std::vector<int8_t> ha((size_t)m * k), hw((size_t)n * k);
	auto refill = [&]() -> int {
		for (auto& v : ha) v = rnd8();
		for (auto& v : hw) v = rnd8();
		CK(hipMemcpy(a, ha.data(), ha.size(), hipMemcpyHostToDevice));
		CK(hipMemcpy(w, hw.data(), hw.size(), hipMemcpyHostToDevice));
		return 0;
	};
	if (refill()) return 1;
	hipStream_t s;
	CK(hipStreamCreate(&s));
	// one eager call on the stream first (the scratch address is set up outside the capture)
	if (sslm_hip_gemm_requant_noalloc(a, w, fold, m, n, k, in_m, in_e, site_m, site_e, codes, me, st, s) != SSLM_OK) {
		printf("eager noalloc call failed\n");
		return 1;
	}
	CK(hipStreamSynchronize(s));
	hipGraph_t graph;
	CK(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
	const sslm_status cst =
	    sslm_hip_gemm_requant_noalloc(a, w, fold, m, n, k, in_m, in_e, site_m, site_e, codes, me, st, s);
	CK(hipStreamEndCapture(s, &graph));
	if (cst != SSLM_OK) {
		printf("captured noalloc call returned %d\n", (int)cst);
		return 1;
	}
	hipGraphExec_t exec;
	CK(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
	std::vector<int8_t> hc((size_t)m * n), hcr((size_t)m * n);
	std::vector<int32_t> hs(m), hsr(m);
	std::vector<int64_t> hm(2 * m), hmr(2 * m);
	int live = 0;
	for (int rep = 0; rep < 3; ++rep) {
		if (rep > 0 && refill()) return 1;  // new inputs in the same buffers
		CK(hipMemset(codes, 0x55, (size_t)m * n));
		CK(hipGraphLaunch(exec, s));
		CK(hipStreamSynchronize(s));
		if (sslm_hip_gemm_requant(a, w, fold, m, n, k, in_m, in_e, site_m, site_e, codes_ref, me_ref, st_ref) !=
		    SSLM_OK) {
			printf("allocating entry failed\n");
			return 1;
		}
		CK(hipMemcpy(hc.data(), codes, hc.size(), hipMemcpyDeviceToHost));
		CK(hipMemcpy(hcr.data(), codes_ref, hcr.size(), hipMemcpyDeviceToHost));
		CK(hipMemcpy(hs.data(), st, m * 4, hipMemcpyDeviceToHost));
		CK(hipMemcpy(hsr.data(), st_ref, m * 4, hipMemcpyDeviceToHost));
		CK(hipMemcpy(hm.data(), me, m * 16, hipMemcpyDeviceToHost));
		CK(hipMemcpy(hmr.data(), me_ref, m * 16, hipMemcpyDeviceToHost));
		for (int t = 0; t < m; ++t) live += hsr[t] == 0;
		if (hc != hcr || hs != hsr || hm != hmr) {
			printf("replay %d differs from the allocating entry\n", rep);
			return 1;
		}
	}
	if (live == 0) {
		printf("every row refused: the check would be vacuous\n");
		return 1;
	}
	CK(hipGraphExecDestroy(exec));
	CK(hipGraphDestroy(graph));
	CK(hipStreamDestroy(s));
	printf("ok (%d live rows)\n", live);
	return 0;
}
