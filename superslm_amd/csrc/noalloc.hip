// The GEMM + requant entry point for callers that cannot allocate device memory (code under HIP
// graph capture, tight serving loops, harnesses that forbid hipMalloc): the same kernels as
// sslm_hip_gemm_requant, with their scratch -- the int32 fold outputs, the per-(16-column tile,
// token) partial maxima, the per-token routing and incoming scales -- in one file-scope device
// array instead of library allocations.
#include <hip/hip_runtime.h>
#include <stdio.h>

#include <mutex>

#include "../../include/sslm_hip.h"
#include "kernels.h"

using namespace sslm;

namespace {

constexpr int kNaMaxM = SSLM_HIP_NOALLOC_MAX_M;
constexpr int kNaMaxN = SSLM_HIP_NOALLOC_MAX_N;
static_assert(kNaMaxN <= kFunnelMaxN, "the funnel kernel covers rows up to kFunnelMaxN");
static_assert(kNaMaxM <= kPartLd, "the partial maxima hold kPartLd tokens per tile");

// scratch layout (byte offsets, each 256-aligned)
constexpr size_t kOffF = 0;                                                  // int32 [M, N]
constexpr size_t kOffMx = kOffF + (size_t)kNaMaxM * kNaMaxN * 4;             // uint32 [tile * kPartLd + t]
constexpr size_t kMxWords = (size_t)(kNaMaxN / 16 - 1) * kPartLd + kNaMaxM;  // highest index + 1
constexpr size_t kOffTok = (kOffMx + kMxWords * 4 + 255) / 256 * 256;        // TokenInfo [M]
constexpr size_t kOffIn = (kOffTok + kNaMaxM * sizeof(TokenInfo) + 255) / 256 * 256;  // Scale [M]
constexpr size_t kScratchBytes = (kOffIn + kNaMaxM * sizeof(Scale) + 255) / 256 * 256;

// Each GPU the library runs on holds its own copy until the process ends.  Host code never uses
// this name as an address: it takes the per-device pointer from hipGetSymbolAddress.
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
void* g_scratch_ptr[kMaxDevices] = {};
std::mutex g_scratch_mu;

// The current device's copy of `scratch`, looked up once per device.
unsigned char* scratch_ptr() {
	int dev = -1;
	if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
	std::lock_guard<std::mutex> lk(g_scratch_mu);
	if (!g_scratch_ptr[dev]) {
		void* p = nullptr;
		const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
		if (e != hipSuccess || !p) {
			fprintf(stderr, "sslm_hip: hipGetSymbolAddress(scratch) failed: %s\n", hipGetErrorString(e));
			return nullptr;
		}
		g_scratch_ptr[dev] = p;
	}
	return (unsigned char*)g_scratch_ptr[dev];
}

// Per-token routing (slot t, position 0), the incoming scale, and a cleared status per token:
// a kernel, so the call records no memset or host copy.
__global__ void k_noalloc_setup(TokenInfo* tok, Scale* in, int32_t* status, int m, int64_t in_m, int64_t in_e) {
	const int t = blockIdx.x * blockDim.x + threadIdx.x;
	if (t >= m) return;
	tok[t] = TokenInfo{0, t, 0};
	in[t] = Scale{in_m, in_e};
	status[t] = 0;
}

}  // namespace

extern "C" {

size_t sslm_hip_noalloc_scratch_bytes(void) { return kScratchBytes; }

sslm_status sslm_hip_gemm_requant_noalloc(const int8_t* a, const int8_t* w, const int32_t* fold, int32_t m, int32_t n,
                                          int32_t k, int64_t in_m, int64_t in_e, int64_t site_m, int64_t site_e,
                                          int8_t* out_codes, int64_t* out_me, int32_t* out_status,
                                          void* stream_handle) {
	hipStream_t stream = (hipStream_t)stream_handle;
	if (!a || !w || !fold || !out_codes || !out_me || !out_status) return SSLM_INVALID_ARGUMENT;
	if (m < 1 || m > kNaMaxM || n < 16 || n > kNaMaxN || n % 16 || k < 16 || k % 16) {
		fprintf(stderr, "sslm_hip_gemm_requant_noalloc: m %d, n %d, k %d outside 1 <= m <= %d, 16 <= n <= %d, "
		        "n and k multiples of 16\n", m, n, k, kNaMaxM, kNaMaxN);
		return SSLM_INVALID_ARGUMENT;
	}
	unsigned char* base = scratch_ptr();
	if (!base) return SSLM_INVALID_ARGUMENT;
	(void)hipGetLastError();  // an error left by an unrelated earlier call is not this call's
	int32_t* f = (int32_t*)(base + kOffF);
	uint32_t* mx = (uint32_t*)(base + kOffMx);
	TokenInfo* tok = (TokenInfo*)(base + kOffTok);
	Scale* in = (Scale*)(base + kOffIn);

	hipLaunchKernelGGL(k_noalloc_setup, dim3((m + 255) / 256), dim3(256), 0, stream, tok, in, out_status, m, in_m, in_e);
	if (hipGetLastError() != hipSuccess) return SSLM_HIP_LAUNCH_FAILED;
	GemmArgs g{};
	g.a = a;
	g.w = w;
	g.M = m;
	g.N = n;
	g.K = k;
	g.lda = k;
	g.epi.tok = tok;
	g.epi.status = out_status;
	g.epi.nseg = 1;
	Segment& sg = g.epi.seg[0];
	sg.n_begin = 0;
	sg.n_end = n;
	sg.mode = kSegFunnel;
	sg.out = f;
	sg.ld_out = n;
	sg.maxpart = mx;
	sg.fold = fold;
	try {
		sslm_launch::gemm(g, stream);
	} catch (const sslm_launch::LaunchRefused&) {
		return SSLM_HIP_LAUNCH_FAILED;
	}
	if (hipGetLastError() != hipSuccess) return SSLM_HIP_LAUNCH_FAILED;
	sslm_launch::FunnelArgs fa{};
	fa.M = m;
	fa.N = n;
	fa.tok = tok;
	fa.f = f;
	fa.ld_f = n;
	fa.maxpart = mx;
	fa.ntiles = n / 16;
	fa.incoming = in;
	fa.site = Scale{site_m, site_e};
	fa.out = out_codes;
	fa.out_scale = (Scale*)out_me;
	fa.layer = 0;
	fa.status = out_status;
	try {
		sslm_launch::funnel(fa, stream);
	} catch (const sslm_launch::LaunchRefused&) {
		return SSLM_HIP_LAUNCH_FAILED;
	}
	if (hipGetLastError() != hipSuccess) return SSLM_HIP_LAUNCH_FAILED;
	return SSLM_OK;
}

}  // extern "C"
