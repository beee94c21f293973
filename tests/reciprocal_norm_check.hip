// Exhaustive device check of reciprocal_norm (superslm_amd/csrc/int_math.h), the reciprocal every
// funnel plan uses on the GPU: for every normalized divisor dn in [2^30, 2^31) it must equal
// reciprocal_div (round_half_up(2^62 / dn), the value the reference's corrected-Newton
// DynamicScaleReciprocal returns, src/intmath.cpp:303-333), which the host tests pin against the
// oracle.  Prints the mismatch count; exit status 0 only when it is zero.
#include <hip/hip_runtime.h>
#include <cstdio>
#include "int_math.h"
using namespace sslm;

__global__ void k_check(unsigned long long* bad, long long* first) {
	const int64_t base = (int64_t)1 << 30;
	unsigned long long nb = 0;
	long long fb = (long long)1 << 40;
	for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < base; i += (int64_t)gridDim.x * blockDim.x) {
		const int64_t dn = base + i;
		if (reciprocal_norm(dn) != reciprocal_div(dn)) {
			++nb;
			fb = fb < dn ? fb : dn;
		}
	}
	if (nb) {
		atomicAdd(bad, nb);
		atomicMin(first, fb);
	}
}

int main() {
	unsigned long long* bad;
	long long* first;
	if (hipMalloc(&bad, 8) != hipSuccess || hipMalloc(&first, 8) != hipSuccess) return 2;
	unsigned long long zb = 0;
	long long zf = (long long)1 << 40;
	if (hipMemcpy(bad, &zb, 8, hipMemcpyHostToDevice) != hipSuccess) return 2;
	if (hipMemcpy(first, &zf, 8, hipMemcpyHostToDevice) != hipSuccess) return 2;
	k_check<<<8192, 256>>>(bad, first);
	if (hipDeviceSynchronize() != hipSuccess) return 2;
	if (hipMemcpy(&zb, bad, 8, hipMemcpyDeviceToHost) != hipSuccess) return 2;
	if (hipMemcpy(&zf, first, 8, hipMemcpyDeviceToHost) != hipSuccess) return 2;
	printf("reciprocal_norm over every dn in [2^30, 2^31): %llu mismatches\n", zb);
	if (zb) printf("first mismatch at dn = %lld\n", zf);
	return zb == 0 ? 0 : 1;
}
