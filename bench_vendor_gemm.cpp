// Reference point for bench.py's prefill GEMM roofline: AMD's own int8 x int8 -> int32 GEMMs
// (hipBLASLt, best of its heuristic's candidates, and rocBLAS gemm_ex) on the projection shapes of
// one 1.5B-shape 512-token prefill chunk, out[M][N] = A[M][K] . W[N][K]^T, each shape over 28
// rotating weight copies as a chunk's 28 layers stream them, timed with HIP events.  Plain GEMMs
// with raw int32 output (no fold, funnel or split planes).  Prints one JSON object.
// Built by __graft_entry__.build() into ./bench_vendor_gemm; bench.py runs it as a child process.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>
#include <rocblas/rocblas.h>
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <string>
#include <vector>

#define CK(x)                                                                                  \
	do {                                                                                       \
		hipError_t e_ = (x);                                                                   \
		if (e_ != hipSuccess) {                                                                \
			fprintf(stderr, "HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);    \
			return 1;                                                                          \
		}                                                                                      \
	} while (0)

int main() {
	struct Shape {
		const char* name;
		int M, N, K;
	} shapes[] = {{"q|k|v", 512, 2048, 1536}, {"o", 512, 1536, 1536}, {"gate|up", 512, 17920, 1536}, {"down", 512, 1536, 8960}};
	const int kCopies = 28, kIters = 5;
	rocblas_handle rb;
	if (rocblas_create_handle(&rb) != rocblas_status_success) return 1;
	hipblasLtHandle_t lt;
	if (hipblasLtCreate(&lt) != HIPBLAS_STATUS_SUCCESS) return 1;
	hipEvent_t e0, e1;
	CK(hipEventCreate(&e0));
	CK(hipEventCreate(&e1));
	const size_t wsz = 64 << 20;
	void* ws;
	CK(hipMalloc(&ws, wsz));
	std::string out = "{\"shapes\": {";
	double sum_lt = 0, sum_rb = 0, ops_layer = 0;
	for (size_t si = 0; si < sizeof(shapes) / sizeof(shapes[0]); ++si) {
		const Shape& s = shapes[si];
		int8_t* A;
		int32_t* C;
		std::vector<int8_t*> W(kCopies);
		CK(hipMalloc(&A, (size_t)s.M * s.K));
		CK(hipMemset(A, 3, (size_t)s.M * s.K));
		for (auto& p : W) {
			CK(hipMalloc(&p, (size_t)s.N * s.K));
			CK(hipMemset(p, 5, (size_t)s.N * s.K));
		}
		CK(hipMalloc(&C, (size_t)s.M * s.N * 4));
		const double ops = 2.0 * s.M * s.N * s.K;
		ops_layer += ops;
		int32_t alpha = 1, beta = 0;
		// mean microseconds per GEMM over kIters passes of the 28 copies (one untimed pass first)
		auto time_pass = [&](auto&& launch) -> double {
			for (int c = 0; c < kCopies; ++c)
				if (!launch(c)) return -1;
			if (hipDeviceSynchronize() != hipSuccess) return -1;
			if (hipEventRecord(e0, 0) != hipSuccess) return -1;
			for (int it = 0; it < kIters; ++it)
				for (int c = 0; c < kCopies; ++c) launch(c);
			if (hipEventRecord(e1, 0) != hipSuccess || hipEventSynchronize(e1) != hipSuccess) return -1;
			float ms = 0;
			if (hipEventElapsedTime(&ms, e0, e1) != hipSuccess) return -1;
			return ms * 1e3 / (kIters * kCopies);
		};
		const double us_rb = time_pass([&](int c) {
			return rocblas_gemm_ex(rb, rocblas_operation_transpose, rocblas_operation_none, s.N, s.M, s.K, &alpha, W[c],
			                       rocblas_datatype_i8_r, s.K, A, rocblas_datatype_i8_r, s.K, &beta, C,
			                       rocblas_datatype_i32_r, s.N, C, rocblas_datatype_i32_r, s.N, rocblas_datatype_i32_r,
			                       rocblas_gemm_algo_standard, 0, 0) == rocblas_status_success;
		});
		// hipBLASLt: column-major C (N x M) = op_T(W as K x N) * (A as K x M)
		hipblasLtMatmulDesc_t md;
		hipblasLtMatmulDescCreate(&md, HIPBLAS_COMPUTE_32I, HIP_R_32I);
		hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
		hipblasLtMatmulDescSetAttribute(md, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta));
		hipblasLtMatmulDescSetAttribute(md, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb));
		hipblasLtMatrixLayout_t la, lb, lc;
		hipblasLtMatrixLayoutCreate(&la, HIP_R_8I, s.K, s.N, s.K);
		hipblasLtMatrixLayoutCreate(&lb, HIP_R_8I, s.K, s.M, s.K);
		hipblasLtMatrixLayoutCreate(&lc, HIP_R_32I, s.N, s.M, s.N);
		hipblasLtMatmulPreference_t pref;
		hipblasLtMatmulPreferenceCreate(&pref);
		hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsz, sizeof(wsz));
		hipblasLtMatmulHeuristicResult_t res[16];
		int nres = 0;
		double us_lt = -1;
		if (hipblasLtMatmulAlgoGetHeuristic(lt, md, la, lb, lc, lc, pref, 16, res, &nres) == HIPBLAS_STATUS_SUCCESS) {
			for (int r = 0; r < nres; ++r) {
				const double us = time_pass([&](int c) {
					return hipblasLtMatmul(lt, md, &alpha, W[c], la, A, lb, &beta, C, lc, C, lc, &res[r].algo, ws, wsz,
					                       0) == HIPBLAS_STATUS_SUCCESS;
				});
				if (us > 0 && (us_lt < 0 || us < us_lt)) us_lt = us;
			}
		}
		hipblasLtMatmulPreferenceDestroy(pref);
		hipblasLtMatrixLayoutDestroy(la);
		hipblasLtMatrixLayoutDestroy(lb);
		hipblasLtMatrixLayoutDestroy(lc);
		hipblasLtMatmulDescDestroy(md);
		sum_lt += us_lt;
		sum_rb += us_rb;
		char buf[512];
		snprintf(buf, sizeof buf,
		         "%s\"%s\": {\"M\": %d, \"N\": %d, \"K\": %d, \"hipblaslt_us\": %.2f, \"hipblaslt_tops\": %.1f, "
		         "\"rocblas_us\": %.2f, \"rocblas_tops\": %.1f}",
		         si ? ", " : "", s.name, s.M, s.N, s.K, us_lt, ops / us_lt / 1e6, us_rb, ops / us_rb / 1e6);
		out += buf;
		for (auto p : W) CK(hipFree(p));
		CK(hipFree(A));
		CK(hipFree(C));
	}
	const double best = std::min(sum_lt, sum_rb);
	char buf[512];
	snprintf(buf, sizeof buf,
	         "}, \"layer_us_hipblaslt\": %.2f, \"layer_us_rocblas\": %.2f, \"pass_tops_best\": %.1f, "
	         "\"pass_frac_of_5000_tops\": %.4f}",
	         sum_lt, sum_rb, ops_layer / best / 1e6, ops_layer / best / 1e6 / 5000.0);
	out += buf;
	printf("%s\n", out.c_str());
	return 0;
}
