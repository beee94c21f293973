// HIP kernels of the SuperSLM integer forward path for gfx950 (CDNA4).
//
// Every kernel computes exactly what the reference CPU path computes (src/matmul.cpp,
// src/intmath.cpp, src/silu_lut.cpp, src/forward/*.cpp); integer sums are order-free, so tiling,
// split-K and wavefront reductions change no bit.  Rejections are reported per sequence slot in a
// status word instead of aborting (the reference's SslmForwardStatus values).
#include <hip/hip_runtime.h>

#include <algorithm>

#include "kernels.h"

namespace sslm {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kBlock = 256;
constexpr int kRowBlock = 1024;  // row kernels: one block per token

// ------------------------------------------------------------------------------------------
// reductions
// ------------------------------------------------------------------------------------------
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
	for (int o = 32; o > 0; o >>= 1) {
		uint64_t w = __shfl_xor(v, o, 64);
		v = w > v ? w : v;
	}
	return v;
}

__device__ __forceinline__ int64_t wave_sum_i64(int64_t v) {
	for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
	return v;
}

__device__ __forceinline__ int64_t wave_max_i64(int64_t v) {
	for (int o = 32; o > 0; o >>= 1) {
		int64_t w = __shfl_xor(v, o, 64);
		v = w > v ? w : v;
	}
	return v;
}

// block-wide reductions over blockDim.x threads; `red` holds blockDim.x/64 (<= 16) slots
__device__ __forceinline__ uint64_t block_max_u64(uint64_t v, uint64_t* red) {
	v = wave_max_u64(v);
	const int w = threadIdx.x >> 6;
	__syncthreads();
	if ((threadIdx.x & 63) == 0) red[w] = v;
	__syncthreads();
	uint64_t r = red[0];
	for (int i = 1; i < (int)(blockDim.x >> 6); ++i) r = red[i] > r ? red[i] : r;
	return r;
}

__device__ __forceinline__ int64_t block_sum_i64(int64_t v, int64_t* red) {
	v = wave_sum_i64(v);
	const int w = threadIdx.x >> 6;
	__syncthreads();
	if ((threadIdx.x & 63) == 0) red[w] = v;
	__syncthreads();
	int64_t r = 0;
	for (int i = 0; i < (int)(blockDim.x >> 6); ++i) r += red[i];
	return r;
}

__device__ __forceinline__ int64_t block_max_i64(int64_t v, int64_t* red) {
	v = wave_max_i64(v);
	const int w = threadIdx.x >> 6;
	__syncthreads();
	if ((threadIdx.x & 63) == 0) red[w] = v;
	__syncthreads();
	int64_t r = red[0];
	for (int i = 1; i < (int)(blockDim.x >> 6); ++i) r = red[i] > r ? red[i] : r;
	return r;
}

// max over tiles [tile0, tile0 + ntiles) of a per-(tile, token) partial array; every thread of
// the block must call it
__device__ __forceinline__ uint64_t reduce_part(const uint32_t* part, int tile0, int ntiles, int t, uint64_t* red) {
	uint64_t m = 0;
	for (int i = threadIdx.x; i < ntiles; i += blockDim.x) {
		const uint64_t v = part[(size_t)(tile0 + i) * kPartLd + t];
		m = v > m ? v : m;
	}
	return block_max_u64(m, red);
}

__device__ __forceinline__ uint32_t sat_abs_u32(int64_t v) {
	uint64_t a = v < 0 ? (uint64_t)0 - (uint64_t)v : (uint64_t)v;
	return a > 0xffffffffull ? 0xffffffffu : (uint32_t)a;
}

__device__ __forceinline__ int32_t sat_i32(int64_t v) {
	return v > kI32Max ? kI32Max : (v < kI32Min ? kI32Min : (int32_t)v);
}

// ------------------------------------------------------------------------------------------
// projection epilogue: WSC1 fold -> LoRA delta -> bias reconcile (forward_sites.cpp:1114-1141)
// ------------------------------------------------------------------------------------------
struct EpiResult {
	int seg;
	int64_t v;
	bool ok;
};

__device__ __forceinline__ EpiResult epi_value(const Epilogue& e, int t, int j, int32_t acc) {
	int si = 0;
	while (si + 1 < e.nseg && j >= e.seg[si].n_end) ++si;
	const Segment& sg = e.seg[si];
	const int jj = j - sg.n_begin;
	const int32_t* f = sg.fold + 3 * jj;
	int64_t v = apply_fold((int64_t)acc, f[0], f[1], f[2]);
	if (sg.lora_b) {
		const int8_t* br = sg.lora_b + (size_t)jj * e.rank;
		const int8_t* ur = sg.lora_u + (size_t)t * kMaxRank;
		int64_t d = 0;
		for (int r = 0; r < e.rank; ++r) d += (int32_t)br[r] * (int32_t)ur[r];
		const int32_t* df = sg.lora_dfold + 3 * jj;
		v += apply_amp_fold(d, df[0], df[1], df[2]);
	}
	bool ok = true;
	if (sg.bias) {
		int64_t term;
		ok = bias_term(sg.bias[jj], e.in_recip[t], e.in_scale[t].e, v, &term);
		if (ok) v += term;
	}
	return EpiResult{si, v, ok};
}

__device__ __forceinline__ void epi_store(const Epilogue& e, const EpiResult& r, int t, int j) {
	const Segment& sg = e.seg[r.seg];
	const int jj = j - sg.n_begin;
	if (sg.mode == kSegWide) {
		((int64_t*)sg.out)[(size_t)t * sg.ld_out + jj] = r.v;
	} else {
		((int32_t*)sg.out)[(size_t)t * sg.ld_out + jj] = sat_i32(r.v);
	}
}

__device__ __forceinline__ v4i load16(const int8_t* p) { return *(const v4i*)p; }

// One output element (token t, channel j) of any GEMM: raw accumulator, argmax key, or the
// projection epilogue; returns the element's contribution to its tile's partial max.
__device__ __forceinline__ void epi_element(const Epilogue& e, int N, int t, int j, int32_t acc, uint64_t* key,
                                            uint32_t* mabs, int* seg) {
	if (e.raw_out) {
		e.raw_out[(size_t)t * N + j] = acc;
	} else if (e.argmax_key) {
		const uint32_t logit = (uint32_t)acc ^ 0x80000000u;
		*key = ((uint64_t)logit << 32) | (uint64_t)(0xffffffffu - (uint32_t)j);
	} else {
		EpiResult r = epi_value(e, t, j, acc);
		if (!r.ok) set_status(e.status, e.tok[t].slot, e.layer, kBiasReconcileProductOutOfDomain);
		epi_store(e, r, t, j);
		*seg = r.seg;
		if (e.seg[r.seg].mode == kSegFunnel) *mabs = sat_abs_u32(r.v);
	}
}

// Reduce over the 16 lanes holding one token's 16 consecutive channels (a 16-column tile; segment
// bounds are multiples of 16) and store the tile's partial: no atomics, one writer per
// (tile, token).  Lane groups of 16 must be converged here.
__device__ __forceinline__ void epi_publish(const Epilogue& e, int tile, int t, bool live, uint64_t key, uint32_t mabs,
                                            int seg) {
	for (int o = 8; o > 0; o >>= 1) {
		uint64_t k2 = __shfl_xor(key, o, 16);
		key = k2 > key ? k2 : key;
		uint32_t m2 = __shfl_xor(mabs, o, 16);
		mabs = m2 > mabs ? m2 : mabs;
	}
	if ((threadIdx.x & 15) == 0 && live) {
		if (e.argmax_key) {
			e.argmax_key[(size_t)tile * kPartLd + t] = key;
		} else if (!e.raw_out && e.seg[seg].mode == kSegFunnel && e.seg[seg].maxpart) {
			e.seg[seg].maxpart[(size_t)tile * kPartLd + t] = mabs;
		}
	}
}

// ------------------------------------------------------------------------------------------
// Streaming decode GEMV (M <= 64): a block of WAVES waves owns 16 output channels; K is walked in
// 128-byte chunks dealt round-robin to the waves.  Per chunk a lane loads 32 contiguous bytes of
// a weight row (a wave covers 16 rows x 128 B) and feeds two v_mfma_i32_16x16x64_i8 with the
// activations loaded in the same lane->k mapping, so the k permutation is identical on both
// operands and the integer sum is exact.  The next chunk is in flight while the current one is
// multiplied.  The waves' partial tiles meet in LDS; no global split, no atomics.
// ------------------------------------------------------------------------------------------
template <int MB, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void k_gemv_stream(GemmArgs g) {
	__shared__ v4i red[WAVES][MB][64];
	const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
	const int col0 = blockIdx.x * 16;
	const int ri = lane & 15, grp = lane >> 4;
	const int C = g.K >> 7;
	const int my_col = col0 + ri;
	const bool col_ok = my_col < g.N;
	const int8_t* wrow = g.w + (size_t)(col_ok ? my_col : 0) * g.K + grp * 32;
	const int8_t* arow[MB];
	bool row_ok[MB];
#pragma unroll
	for (int mb = 0; mb < MB; ++mb) {
		const int r = mb * 16 + ri;
		row_ok[mb] = r < g.M;
		arow[mb] = g.a + (size_t)(row_ok[mb] ? r : 0) * g.lda + grp * 32;
	}
	v4i acc[MB];
#pragma unroll
	for (int mb = 0; mb < MB; ++mb) acc[mb] = v4i{0, 0, 0, 0};
	const v4i z = v4i{0, 0, 0, 0};
	int c = wave;
	v4i b0 = z, b1 = z, a0[MB], a1[MB];
#pragma unroll
	for (int mb = 0; mb < MB; ++mb) a0[mb] = a1[mb] = z;
	if (c < C) {
		const int8_t* wp = wrow + (size_t)c * 128;
		b0 = col_ok ? load16(wp) : z;
		b1 = col_ok ? load16(wp + 16) : z;
#pragma unroll
		for (int mb = 0; mb < MB; ++mb) {
			a0[mb] = row_ok[mb] ? load16(arow[mb] + (size_t)c * 128) : z;
			a1[mb] = row_ok[mb] ? load16(arow[mb] + (size_t)c * 128 + 16) : z;
		}
	}
	while (c < C) {
		const int cn = c + WAVES;
		v4i nb0 = z, nb1 = z, na0[MB], na1[MB];
#pragma unroll
		for (int mb = 0; mb < MB; ++mb) na0[mb] = na1[mb] = z;
		if (cn < C) {
			const int8_t* wp = wrow + (size_t)cn * 128;
			nb0 = col_ok ? load16(wp) : z;
			nb1 = col_ok ? load16(wp + 16) : z;
#pragma unroll
			for (int mb = 0; mb < MB; ++mb) {
				na0[mb] = row_ok[mb] ? load16(arow[mb] + (size_t)cn * 128) : z;
				na1[mb] = row_ok[mb] ? load16(arow[mb] + (size_t)cn * 128 + 16) : z;
			}
		}
#pragma unroll
		for (int mb = 0; mb < MB; ++mb) {
			acc[mb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0[mb], b0, acc[mb], 0, 0, 0);
			acc[mb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1[mb], b1, acc[mb], 0, 0, 0);
		}
		c = cn;
		b0 = nb0;
		b1 = nb1;
#pragma unroll
		for (int mb = 0; mb < MB; ++mb) {
			a0[mb] = na0[mb];
			a1[mb] = na1[mb];
		}
	}
#pragma unroll
	for (int mb = 0; mb < MB; ++mb) red[wave][mb][lane] = acc[mb];
	__syncthreads();
	// wave w finishes row block mb = w (and w + WAVES, ... when MB > WAVES)
	const Epilogue& e = g.epi;
	const int j = col0 + ri;
	for (int mb = wave; mb < MB; mb += WAVES) {
		v4i tot = red[0][mb][lane];
		for (int w = 1; w < WAVES; ++w) {
			const v4i x = red[w][mb][lane];
			tot[0] += x[0];
			tot[1] += x[1];
			tot[2] += x[2];
			tot[3] += x[3];
		}
#pragma unroll
		for (int v = 0; v < 4; ++v) {
			const int t = mb * 16 + grp * 4 + v;
			uint64_t key = 0;
			uint32_t mabs = 0;
			int seg = 0;
			if (t < g.M && j < g.N) epi_element(e, g.N, t, j, tot[v], &key, &mabs, &seg);
			epi_publish(e, blockIdx.x, t, t < g.M && col0 < g.N, key, mabs, seg);
		}
	}
}

// ------------------------------------------------------------------------------------------
// tiled MFMA GEMM for prefill chunks: 128x128 block tile, BK=64, LDS-staged A and B,
// v_mfma_i32_32x32x32_i8, each wave a 64x64 sub-tile (2x2 MFMA tiles).  The accumulators go
// through LDS for the epilogue so every thread finishes whole 16-column tile rows.
// ------------------------------------------------------------------------------------------
constexpr int kBM = 128, kBN = 128, kBK = 64, kLdsStride = 80;  // padded row stride (bytes)

__global__ __launch_bounds__(kBlock) void k_gemm_tiled(GemmArgs g) {
	__shared__ __attribute__((aligned(16))) int8_t smem[2 * (kBM + kBN) * kLdsStride];
	int8_t* sa0 = smem;
	int8_t* sb0 = smem + kBM * kLdsStride;
	const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
	const int m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;
	const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
	v16i acc00, acc01, acc10, acc11;
	for (int v = 0; v < 16; ++v) acc00[v] = acc01[v] = acc10[v] = acc11[v] = 0;

	const int chunk0 = threadIdx.x, chunk1 = threadIdx.x + kBlock;
	const int r0 = chunk0 >> 2, kc0 = (chunk0 & 3) * 16;
	const int r1 = chunk1 >> 2, kc1 = (chunk1 & 3) * 16;
	v4i ra0, ra1, rb0, rb1;
	const v4i z = v4i{0, 0, 0, 0};
	auto gload = [&](int k0) {
		ra0 = (m0 + r0 < g.M && k0 + kc0 < g.K) ? load16(g.a + (size_t)(m0 + r0) * g.lda + k0 + kc0) : z;
		ra1 = (m0 + r1 < g.M && k0 + kc1 < g.K) ? load16(g.a + (size_t)(m0 + r1) * g.lda + k0 + kc1) : z;
		rb0 = (n0 + r0 < g.N && k0 + kc0 < g.K) ? load16(g.w + (size_t)(n0 + r0) * g.K + k0 + kc0) : z;
		rb1 = (n0 + r1 < g.N && k0 + kc1 < g.K) ? load16(g.w + (size_t)(n0 + r1) * g.K + k0 + kc1) : z;
	};
	auto sstore = [&](int buf) {
		int8_t* sa = smem + buf * (kBM + kBN) * kLdsStride;
		int8_t* sb = sa + kBM * kLdsStride;
		*(v4i*)&sa[r0 * kLdsStride + kc0] = ra0;
		*(v4i*)&sa[r1 * kLdsStride + kc1] = ra1;
		*(v4i*)&sb[r0 * kLdsStride + kc0] = rb0;
		*(v4i*)&sb[r1 * kLdsStride + kc1] = rb1;
	};
	gload(0);
	sstore(0);
	__syncthreads();
	const int nk = (g.K + kBK - 1) / kBK;
	for (int it = 0; it < nk; ++it) {
		const int buf = it & 1;
		const int8_t* sa = smem + buf * (kBM + kBN) * kLdsStride;
		const int8_t* sb = sa + kBM * kLdsStride;
		if (it + 1 < nk) gload((it + 1) * kBK);
#pragma unroll
		for (int ks = 0; ks < 2; ++ks) {  // two K=32 MFMA steps per BK=64
			const int kk = ks * 32 + (lane >> 5) * 16;
			const v4i a0 = *(const v4i*)&sa[(wm + (lane & 31)) * kLdsStride + kk];
			const v4i a1 = *(const v4i*)&sa[(wm + 32 + (lane & 31)) * kLdsStride + kk];
			const v4i b0 = *(const v4i*)&sb[(wn + (lane & 31)) * kLdsStride + kk];
			const v4i b1 = *(const v4i*)&sb[(wn + 32 + (lane & 31)) * kLdsStride + kk];
			acc00 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, b0, acc00, 0, 0, 0);
			acc01 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, b1, acc01, 0, 0, 0);
			acc10 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, b0, acc10, 0, 0, 0);
			acc11 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, b1, acc11, 0, 0, 0);
		}
		if (it + 1 < nk) sstore(buf ^ 1);
		__syncthreads();
	}
	(void)sa0;
	(void)sb0;
	// accumulators -> LDS as int32 [128 rows][128 cols] in two passes of 64 rows (32 KB each)
	int32_t* ct = (int32_t*)smem;  // 2 * 256 * 80 = 40 KB >= 64 x 128 x 4 = 32 KB
	const Epilogue& e = g.epi;
	for (int half = 0; half < 2; ++half) {
		__syncthreads();
		if ((wave >> 1) == half) {
			// 32x32 layout: lane holds column lane%32, rows 8*(v/4) + 4*(lane/32) + v%4
			for (int v = 0; v < 16; ++v) {
				const int rr = (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3);
				const int cc = lane & 31;
				ct[(rr) * kBN + wn + cc] = acc00[v];
				ct[(rr) * kBN + wn + 32 + cc] = acc01[v];
				ct[(32 + rr) * kBN + wn + cc] = acc10[v];
				ct[(32 + rr) * kBN + wn + 32 + cc] = acc11[v];
			}
		}
		__syncthreads();
		// thread -> (row, 16-column group, column): 64 rows x 8 groups x 16 = 8192 elements
		for (int idx = threadIdx.x; idx < 64 * kBN; idx += kBlock) {
			const int rr = idx >> 7, cc = idx & 127;
			const int t = m0 + half * 64 + rr, col = n0 + cc;
			uint64_t key = 0;
			uint32_t mabs = 0;
			int seg = 0;
			if (t < g.M && col < g.N) epi_element(e, g.N, t, col, ct[rr * kBN + cc], &key, &mabs, &seg);
			epi_publish(e, col >> 4, t, t < g.M && (col & ~15) < g.N, key, mabs, seg);
		}
	}
}

// ------------------------------------------------------------------------------------------
// row kernels (one 256-thread block per token)
// ------------------------------------------------------------------------------------------

// forward_sites.cpp:763-787 -- embed row -> funnel ("embed" site, empty incoming)
__global__ __launch_bounds__(kRowBlock) void k_embed(const int32_t* tokens, const int8_t* embed_w, int H, int vocab,
                                                  Scale site, int8_t* out_codes, const int32_t* out_idx,
                                                  Scale* out_scale, const int32_t* scale_idx, const TokenInfo* tok,
                                                  int32_t* status) {
	__shared__ uint64_t red[16];
	__shared__ FunnelPlan plan;
	__shared__ int32_t st;
	const int t = blockIdx.x;
	const int32_t id = tokens[t];
	if (id < 0 || id >= vocab) {
		if (threadIdx.x == 0) set_status(status, tok[t].slot, 0, kTokenIdOutOfRange);
		return;
	}
	const int8_t* row = embed_w + (size_t)id * H;
	uint64_t mx = 0;
	for (int i = threadIdx.x; i < H; i += kRowBlock) {
		int64_t v = row[i];
		uint64_t a = v < 0 ? -v : v;
		mx = a > mx ? a : mx;
	}
	mx = block_max_u64(mx, red);
	if (threadIdx.x == 0) st = funnel_plan(mx, nullptr, 0, site, &plan);
	__syncthreads();
	if (st != kOk) {
		if (threadIdx.x == 0) set_status(status, tok[t].slot, 0, st);
		return;
	}
	int8_t* out = out_codes + (size_t)out_idx[t] * H;
	for (int i = threadIdx.x; i < H; i += kRowBlock) out[i] = requant_code_small(row[i], (uint64_t)plan.r, plan.s);
	if (threadIdx.x == 0) out_scale[scale_idx[t]] = plan.out;
}

// forward_sites.cpp:410-459 -- the RMSNorm site body, shared by the fused row kernels.
// Writes codes to `out` (row of the current token) and returns the status.
__device__ int32_t rmsnorm_row(const int8_t* h, const int32_t* g, int H, Scale site, int8_t* out, Scale* out_scale,
                               int64_t* out_recip, uint64_t* red_u, int64_t* red_s) {
	__shared__ int64_t s_root;
	__shared__ int64_t fd[256];  // floor((h << 32) / root) for every int8 h
	__shared__ FunnelPlan plan;
	__shared__ int32_t st;
	int64_t ss = 0;
	for (int i = threadIdx.x; i < H; i += blockDim.x) ss += (int64_t)h[i] * h[i];
	ss = block_sum_i64(ss, red_s);
	if (threadIdx.x == 0) {
		int64_t root = isqrt(floor_div(ss << 32, (int64_t)H));
		s_root = root > 1 ? root : 1;
	}
	__syncthreads();
	const int64_t root = s_root;
	if (threadIdx.x < 256) {
		const int64_t hv = (int64_t)threadIdx.x - 128;
		const int64_t a = hv << 32;
		fd[threadIdx.x] = a >= 0 ? div_floor_pos(a, root) : -div_floor_pos(-a + root - 1, root);
	}
	__syncthreads();
	uint64_t mx = 0;
	for (int i = threadIdx.x; i < H; i += blockDim.x) {
		int64_t w = fd[(int)h[i] + 128] * (int64_t)g[i];
		uint64_t a = w < 0 ? (uint64_t)0 - (uint64_t)w : (uint64_t)w;
		mx = a > mx ? a : mx;
	}
	mx = block_max_u64(mx, red_u);
	if (threadIdx.x == 0) st = funnel_plan(mx, nullptr, 0, site, &plan);
	__syncthreads();
	if (st != kOk) return st;
	for (int i = threadIdx.x; i < H; i += blockDim.x) {
		int64_t w = fd[(int)h[i] + 128] * (int64_t)g[i];
		out[i] = requant_code_small(w, (uint64_t)plan.r, plan.s);
	}
	if (threadIdx.x == 0) {
		*out_scale = plan.out;
		if (out_recip) *out_recip = fits_i32(plan.out.m) ? reciprocal_fast(plan.out.m) : 0;
	}
	__syncthreads();
	return kOk;
}

__global__ __launch_bounds__(kRowBlock) void k_rmsnorm(sslm_launch::RowNormArgs a, int H, const TokenInfo* tok,
                                                    int32_t* status, int32_t layer) {
	__shared__ uint64_t red_u[16];
	__shared__ int64_t red_s[16];
	const int t = blockIdx.x;
	if (status[tok[t].slot] != 0) return;
	const int8_t* h = a.in_codes + (size_t)a.in_idx[t] * a.ld_in;
	int32_t st = rmsnorm_row(h, a.gain, H, a.site, a.out + (size_t)t * H, &a.out_scale[t],
	                         a.out_recip ? &a.out_recip[t] : nullptr, red_u, red_s);
	if (threadIdx.x == 0) set_status(status, tok[t].slot, layer, st);
}

// q funnel + RoPE(q); K/V landing, RoPE(K), KV write (forward_sites.cpp:1281-1418, :1748-1787)
__global__ __launch_bounds__(kRowBlock) void k_qkv_post(sslm_launch::QkvPostArgs a) {
	__shared__ FunnelPlan plan;
	__shared__ int32_t st;
	__shared__ unsigned long long sat_block;
	const int t = blockIdx.x;
	const TokenInfo ti = a.tok[t];
	if (a.status[ti.slot] != 0) return;
	const int H = a.H, D = a.D, pairs = D / 2;
	const int64_t pos = ti.pos;
	__shared__ uint64_t red_u[16];
	const uint64_t mx = reduce_part(a.q_maxpart, 0, H / 16, t, red_u);
	if (threadIdx.x == 0) {
		sat_block = 0;
		const Scale inc = a.in_scale[t];
		st = funnel_plan(mx, &inc, 1, a.q_site, &plan);
		if (st == kOk && (pos < 0 || pos >= a.cap)) st = kPositionOverCap;
	}
	__syncthreads();
	if (st != kOk) {
		if (threadIdx.x == 0) set_status(a.status, ti.slot, a.layer, st);
		return;
	}
	const int64_t* cs = a.rope_cos + pos * pairs;
	const int64_t* sn = a.rope_sin + pos * pairs;
	// q: codes of pair (2i, 2i+1), rotated, clamped
	const int32_t* qf = a.q_f + (size_t)t * H;
	for (int p = threadIdx.x; p < H / 2; p += kRowBlock) {
		const int i = p % pairs;
		const int32_t x = requant_code_small(qf[2 * p], (uint64_t)plan.r, plan.s);
		const int32_t y = requant_code_small(qf[2 * p + 1], (uint64_t)plan.r, plan.s);
		int64_t xr, yr;
		rope_pair(x, y, (int32_t)cs[i], (int32_t)sn[i], &xr, &yr);
		a.q_rot[(size_t)t * H + 2 * p] = (int8_t)clamp_code(xr);
		a.q_rot[(size_t)t * H + 2 * p + 1] = (int8_t)clamp_code(yr);
	}
	if (threadIdx.x == 0) a.q_scale[t] = plan.out;
	// K/V landing: LandingRescale at the normed scale, per kv head
	const Scale ns = a.in_scale[t];
	const int KVH = a.NKV * D;
	const int64_t* kv = a.kv_f + (size_t)t * 2 * KVH;
	int8_t* blk = a.kv_pool + (int64_t)ti.block * a.block_bytes;
	const int64_t half = a.cap * (int64_t)KVH;
	int8_t* kstore = blk + (int64_t)a.layer * half * 2;
	int8_t* vstore = kstore + half;
	unsigned long long sat = 0;
	for (int p = threadIdx.x; p < KVH / 2; p += kRowBlock) {
		const int h = (2 * p) / D;
		const int i = p % pairs;
		const int64_t k_e = composed_exponent(ns.e, a.e_t_k[h]);
		bool c0, c1, x0, x1;
		const int64_t k0 = clamp_code(landing_rescale(kv[2 * p], ns.m, a.r_t_k[h], k_e, &c0, &x0));
		const int64_t k1 = clamp_code(landing_rescale(kv[2 * p + 1], ns.m, a.r_t_k[h], k_e, &c1, &x1));
		sat += (unsigned long long)c0 + (unsigned long long)c1;
		int64_t xr, yr;
		rope_pair((int32_t)k0, (int32_t)k1, (int32_t)cs[i], (int32_t)sn[i], &xr, &yr);
		int8_t* krow = kstore + ((int64_t)h * a.cap + pos) * D;
		krow[2 * i] = (int8_t)clamp_code(xr);
		krow[2 * i + 1] = (int8_t)clamp_code(yr);
		const int64_t v_e = composed_exponent(ns.e, a.e_t_v[h]);
		const int64_t* vv = kv + KVH;
		int8_t* vrow = vstore + ((int64_t)h * a.cap + pos) * D;
		bool c2, c3;
		vrow[2 * i] = (int8_t)clamp_code(landing_rescale(vv[2 * p], ns.m, a.r_t_v[h], v_e, &c2, &x0));
		vrow[2 * i + 1] = (int8_t)clamp_code(landing_rescale(vv[2 * p + 1], ns.m, a.r_t_v[h], v_e, &c3, &x1));
		sat += (unsigned long long)c2 + (unsigned long long)c3;
	}
	if (sat) atomicAdd(&sat_block, sat);
	__syncthreads();
	if (threadIdx.x == 0 && sat_block) atomicAdd(&a.sat[ti.slot], sat_block);
}

// Attention for one (token, kv head): the group's query heads against positions [0, pos]
// (forward_sites.cpp:1791-1905).  Scores/exps/probabilities live in LDS when they fit, else in
// the per-launch global scratch.
__global__ __launch_bounds__(kBlock) void k_attention(sslm_launch::AttnArgs a, int use_lds) {
	extern __shared__ int64_t dyn[];
	__shared__ int64_t red_s[kBlock / 64];
	__shared__ uint64_t red_u[kBlock / 64];
	__shared__ int64_t c_qln2, c_qb, c_qc, c_M;
	__shared__ int32_t st;
	__shared__ int64_t rowmax[16];
	__shared__ int64_t rowsum[16];
	const int kvh = blockIdx.x, t = blockIdx.y;
	const TokenInfo ti = a.tok[t];
	if (a.status[ti.slot] != 0) return;
	const int D = a.D, group = a.NH / a.NKV;
	const int64_t width = ti.pos + 1;
	if (threadIdx.x == 0) {
		st = kOk;
		const Scale qs = a.q_scale[t];
		const int64_t km = a.khead_m[kvh], ke = a.khead_e[kvh];
		if (!fits_i32(qs.m) || !fits_i32(km)) {
			st = kCarriedScaleMantissaOutOfDomain;
		} else {
			const Scale sm = combine_scale(qs, Scale{km, ke});
			if (!fits_i32(sm.m)) {
				st = kCarriedScaleMantissaOutOfDomain;
			} else {
				int64_t ql, qb, qc;
				if (iexp_scale_constants(sm.m, sm.e, a.ln2_q, a.b_q, a.ca_q, &ql, &qb, &qc) != 0) {
					st = kIExpScaleDerivationOutOfDomain;
				} else {
					st = check_softmax_width(qb, qc, width);
					c_qln2 = ql;
					c_qb = qb;
					c_qc = qc;
					c_M = softmax_ceiling(qb, qc);
				}
			}
		}
	}
	__syncthreads();
	if (st != kOk) {
		if (threadIdx.x == 0) set_status(a.status, ti.slot, a.layer, st);
		return;
	}
	int64_t* sc = use_lds ? dyn : a.scratch + ((int64_t)t * a.NH + (int64_t)kvh * group) * a.cap;
	const int8_t* blk = a.kv_pool + (int64_t)ti.block * a.block_bytes;
	const int64_t half = a.cap * (int64_t)a.NKV * D;
	const int8_t* kbase = blk + (int64_t)a.layer * half * 2 + (int64_t)kvh * a.cap * D;
	const int8_t* vbase = kbase + half;
	const int8_t* q = a.q_rot + (size_t)t * a.H + (size_t)kvh * group * D;
	// pass 1: scores (int32-exact dots, widened) -- 8 lanes per position, 16 bytes each
	const int sub = threadIdx.x & 7;
	for (int64_t p0 = threadIdx.x >> 3; p0 < width; p0 += kBlock / 8) {
		const int8_t* kr = kbase + p0 * D;
		for (int g = 0; g < group; ++g) {
			int32_t acc = 0;
			for (int d = sub * 4; d < D; d += 32) {
				const int32_t kw = *(const int32_t*)(kr + d);
				const int32_t qw = *(const int32_t*)(q + g * D + d);
				acc = __builtin_amdgcn_sdot4(qw, kw, acc, false);
			}
			acc += __shfl_xor(acc, 1, 8);
			acc += __shfl_xor(acc, 2, 8);
			acc += __shfl_xor(acc, 4, 8);
			if (sub == 0) sc[(int64_t)g * a.cap + p0] = acc;
		}
	}
	__syncthreads();
	// pass 2: row max per query head
	for (int g = 0; g < group; ++g) {
		int64_t mx = INT64_MIN;
		for (int64_t p = threadIdx.x; p < width; p += kBlock) mx = max(mx, sc[(int64_t)g * a.cap + p]);
		mx = block_max_i64(mx, red_s);
		if (threadIdx.x == 0) rowmax[g] = mx;
		__syncthreads();
	}
	// pass 3: i-exp values (SoftmaxRowQ15, intmath.cpp:853-889) and the row sums
	int refused = 0;
	for (int g = 0; g < group; ++g) {
		int64_t sum = 0;
		const int64_t mx = rowmax[g];
		for (int64_t p = threadIdx.x; p < width; p += kBlock) {
			int64_t v = iexp_element(sc[(int64_t)g * a.cap + p] - mx, c_qln2, c_qb, c_qc, c_M);
			if (v < 0) {
				refused = 1;
				v = 0;
			}
			sc[(int64_t)g * a.cap + p] = v;
			sum += v;
		}
		sum = block_sum_i64(sum, red_s);
		if (threadIdx.x == 0) rowsum[g] = sum;
		__syncthreads();
	}
	uint64_t anyref = block_max_u64((uint64_t)refused, red_u);
	if (anyref) {
		if (threadIdx.x == 0) set_status(a.status, ti.slot, a.layer, kSoftmaxKernelRefusedAfterGateAccepted);
		return;
	}
	// pass 4: Q15 probabilities p = (e << 15) / max(total, 1)
	for (int g = 0; g < group; ++g) {
		const int64_t denom = rowsum[g] > 1 ? rowsum[g] : 1;
		for (int64_t p = threadIdx.x; p < width; p += kBlock) {
			const int64_t e = sc[(int64_t)g * a.cap + p];
			sc[(int64_t)g * a.cap + p] = div_floor_pos(e << 15, denom);
		}
	}
	__syncthreads();
	// pass 5: context = sum_p prob * V[p] (int32-exact: sum of probs <= 2^15), per-head ctx fold
	uint64_t mabs = 0;
	for (int idx = threadIdx.x; idx < group * D; idx += kBlock) {
		const int g = idx / D, d = idx % D;
		int32_t acc = 0;
		const int64_t* pr = sc + (int64_t)g * a.cap;
		for (int64_t p = 0; p < width; ++p) acc += (int32_t)pr[p] * (int32_t)vbase[p * D + d];
		const int h = kvh * group + g;
		const int32_t* cf = a.ctx_fold + 3 * h;
		const int64_t f = apply_fold(acc, cf[0], cf[1], cf[2]);
		a.ctx_f[(size_t)t * a.H + (size_t)h * D + d] = sat_i32(f);
		uint64_t ab = f < 0 ? (uint64_t)0 - (uint64_t)f : (uint64_t)f;
		mabs = ab > mabs ? ab : mabs;
	}
	mabs = block_max_u64(mabs, red_u);
	if (threadIdx.x == 0) a.ctx_maxpart[(size_t)kvh * kPartLd + t] = mabs > 0xffffffffull ? 0xffffffffu : (uint32_t)mabs;
}

// funnel over an int32 fold-output row (checked_chain_funnel.cpp:257-364)
__global__ __launch_bounds__(kRowBlock) void k_funnel(sslm_launch::FunnelArgs a) {
	__shared__ FunnelPlan plan;
	__shared__ int32_t st;
	const int t = blockIdx.x;
	const int slot = a.tok[t].slot;
	__shared__ uint64_t red_u[16];
	if (a.status[slot] != 0) return;
	const uint64_t mx = reduce_part(a.maxpart, 0, a.ntiles, t, red_u);
	if (threadIdx.x == 0) {
		Scale inc;
		if (a.incoming) inc = a.incoming[t];
		st = funnel_plan(mx, a.incoming ? &inc : nullptr, a.incoming ? 1 : 0, a.site, &plan);
	}
	__syncthreads();
	if (st != kOk) {
		if (threadIdx.x == 0) set_status(a.status, slot, a.layer, st);
		return;
	}
	const int32_t* f = a.f + (size_t)t * a.ld_f;
	for (int i = threadIdx.x; i < a.N; i += kRowBlock) a.out[(size_t)t * a.N + i] = requant_code_small(f[i], (uint64_t)plan.r, plan.s);
	if (threadIdx.x == 0) a.out_scale[t] = plan.out;
}

// projection funnel -> residual reconcile -> (optional) RMSNorm, all on one token's row
// (forward_sites.cpp:871-989 residual; :410-459 norm)
__global__ __launch_bounds__(kRowBlock) void k_residual_norm(sslm_launch::ResidualArgs a) {
	__shared__ FunnelPlan bplan, rplan;
	__shared__ int32_t st;
	__shared__ int64_t r_h;
	__shared__ uint64_t red_u[16];
	__shared__ int64_t red_s[16];
	const int t = blockIdx.x;
	const int slot = a.tok[t].slot;
	const int H = a.H;
	if (a.status[slot] != 0) return;
	const int8_t* stream = a.stream + (size_t)a.stream_idx[t] * H;
	const Scale ss = a.stream_scale[a.stream_idx[t]];
	const uint64_t bmx = reduce_part(a.branch_maxpart, 0, H / 16, t, red_u);
	if (threadIdx.x == 0) {
		const Scale inc = a.branch_in[t];
		st = funnel_plan(bmx, &inc, 1, a.branch_site, &bplan);
		if (st == kOk && !fits_i32(ss.m)) st = kCarriedScaleMantissaOutOfDomain;
		if (st == kOk) r_h = reciprocal_fast(ss.m);
	}
	__syncthreads();
	if (st != kOk) {
		if (threadIdx.x == 0) set_status(a.status, slot, a.layer, st);
		return;
	}
	const Scale bs = bplan.out;
	const int64_t k = composed_exponent(bs.e, ss.e);
	const int32_t* bf = a.branch_f + (size_t)t * H;
	uint64_t mx = 0;
	int bad = 0;
	for (int i = threadIdx.x; i < H; i += kRowBlock) {
		const int8_t code = requant_code_small(bf[i], (uint64_t)bplan.r, bplan.s);
		bool cl, ex;
		const int64_t rec = landing_rescale(code, bs.m, r_h, k, &cl, &ex);
		if (ex) {
			bad = 1;
			continue;
		}
		const int64_t w = rec + stream[i];
		const uint64_t ab = w < 0 ? (uint64_t)0 - (uint64_t)w : (uint64_t)w;
		mx = ab > mx ? ab : mx;
	}
	const uint64_t anybad = block_max_u64((uint64_t)bad, red_u);
	mx = block_max_u64(mx, red_u);
	if (threadIdx.x == 0) {
		if (anybad) st = kResidualReconciliationMagnitudeOutOfDomain;
		else st = funnel_plan(mx, &ss, 1, a.res_site, &rplan);
	}
	__syncthreads();
	if (st != kOk) {
		if (threadIdx.x == 0) set_status(a.status, slot, a.layer, st);
		return;
	}
	// `out` never aliases `stream` (the host routes attn_stream and the committed stream through
	// distinct buffers), so codes are written as they are formed.
	int8_t* out = a.out_stream + (size_t)a.out_idx[t] * H;
	for (int i = threadIdx.x; i < H; i += kRowBlock) {
		const int8_t code = requant_code_small(bf[i], (uint64_t)bplan.r, bplan.s);
		bool cl, ex;
		const int64_t w = landing_rescale(code, bs.m, r_h, k, &cl, &ex) + stream[i];
		out[i] = requant_code_small(w, (uint64_t)rplan.r, rplan.s);
	}
	if (threadIdx.x == 0) a.out_stream_scale[a.out_idx[t]] = rplan.out;
	__syncthreads();
	if (a.gain) {
		const int32_t st2 = rmsnorm_row(out, a.gain, H, a.norm_site, a.norm_out + (size_t)t * H, &a.norm_scale[t],
		                                a.norm_recip ? &a.norm_recip[t] : nullptr, red_u, red_s);
		if (threadIdx.x == 0) set_status(a.status, slot, a.layer, st2);
	}
}

// gate/up funnels -> MlpActSite (forward_sites.cpp:796-864) -> act funnel
__global__ __launch_bounds__(kRowBlock) void k_mlp_act(sslm_launch::ActArgs a) {
	__shared__ FunnelPlan gp, up, ap;
	__shared__ int32_t st;
	__shared__ uint64_t red_u[16];
	const int t = blockIdx.x;
	const int slot = a.tok[t].slot;
	const int I = a.I;
	if (a.status[slot] != 0) return;
	const uint64_t gm = reduce_part(a.gu_maxpart, 0, I / 16, t, red_u);
	const uint64_t um = reduce_part(a.gu_maxpart, I / 16, I / 16, t, red_u);
	if (threadIdx.x == 0) {
		const Scale inc = a.in_scale[t];
		st = funnel_plan(gm, &inc, 1, a.gate_site, &gp);
		if (st == kOk) st = funnel_plan(um, &inc, 1, a.up_site, &up);
		if (st == kOk) st = check_silu_scale(gp.out.m, gp.out.e);
	}
	__syncthreads();
	if (st != kOk) {
		if (threadIdx.x == 0) set_status(a.status, slot, a.layer, st);
		return;
	}
	const Scale gs = gp.out;
	const int32_t* gf = a.gu_f + (size_t)t * 2 * I;
	const int32_t* uf = gf + I;
	uint64_t mx = 0;
	for (int i = threadIdx.x; i < I; i += kRowBlock) {
		const int8_t gc = requant_code_small(gf[i], (uint64_t)gp.r, gp.s);
		const int8_t uc = requant_code_small(uf[i], (uint64_t)up.r, up.s);
		const int32_t sig = silu_sigmoid_q15(a.silu, gc, gs.m, (int)gs.e);
		const int64_t w = (int64_t)gc * sig * (int64_t)uc;
		const uint64_t ab = w < 0 ? (uint64_t)0 - (uint64_t)w : (uint64_t)w;
		mx = ab > mx ? ab : mx;
	}
	mx = block_max_u64(mx, red_u);
	if (threadIdx.x == 0) {
		const Scale inc2[2] = {gp.out, up.out};
		st = funnel_plan(mx, inc2, 2, a.act_site, &ap);
	}
	__syncthreads();
	if (st != kOk) {
		if (threadIdx.x == 0) set_status(a.status, slot, a.layer, st);
		return;
	}
	for (int i = threadIdx.x; i < I; i += kRowBlock) {
		const int8_t gc = requant_code_small(gf[i], (uint64_t)gp.r, gp.s);
		const int8_t uc = requant_code_small(uf[i], (uint64_t)up.r, up.s);
		const int32_t sig = silu_sigmoid_q15(a.silu, gc, gs.m, (int)gs.e);
		const int64_t w = (int64_t)gc * sig * (int64_t)uc;
		a.act[(size_t)t * I + i] = requant_code_small(w, (uint64_t)ap.r, ap.s);
	}
	if (threadIdx.x == 0) a.act_scale[t] = ap.out;
}

// LoRA intermediate (forward_sites.cpp:1066-1086): u[k] = clamp(amp_fold(A[k] . x))
__global__ __launch_bounds__(kBlock) void k_lora_u(sslm_launch::LoraUArgs a) {
	const int t = blockIdx.x;
	const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
	const int8_t* x = a.x + (size_t)t * a.K;
	for (int task = wave; task < a.nproj * a.rank; task += kBlock / 64) {
		const int p = task / a.rank, r = task % a.rank;
		const int8_t* arow = a.a[p] + (size_t)r * a.K;
		int64_t acc = 0;
		for (int k = lane; k < a.K; k += 64) acc += (int32_t)arow[k] * (int32_t)x[k];
		acc = wave_sum_i64(acc);
		if (lane == 0) {
			const int32_t* f = a.ufold[p] + 3 * r;
			a.u[p][(size_t)t * kMaxRank + r] = (int8_t)clamp_code(apply_amp_fold(acc, f[0], f[1], f[2]));
		}
	}
}

// lowest-index argmax (forward_sites.cpp:2427-2437) from per-tile keys: the key orders by
// logit, then by the complement of the index, so the maximum key is the lowest maximal index
__global__ __launch_bounds__(kBlock) void k_argmax_finalize(const unsigned long long* keys, int ntiles,
                                                            int32_t* out) {
	__shared__ uint64_t red[16];
	const int t = blockIdx.x;
	uint64_t k = 0;
	for (int i = threadIdx.x; i < ntiles; i += blockDim.x) {
		const uint64_t v = keys[(size_t)i * kPartLd + t];
		k = v > k ? v : k;
	}
	k = block_max_u64(k, red);
	if (threadIdx.x == 0) out[t] = (int32_t)(0xffffffffu - (uint32_t)(k & 0xffffffffull));
}

}  // namespace sslm

// ------------------------------------------------------------------------------------------
// launch wrappers
// ------------------------------------------------------------------------------------------
namespace sslm_launch {

template <int MB>
static void launch_gemv(const GemmArgs& g, int waves, hipStream_t s) {
	dim3 grid((g.N + 15) / 16);
	if (waves >= 16) hipLaunchKernelGGL((k_gemv_stream<MB, 16>), grid, dim3(64 * 16), 0, s, g);
	else if (waves >= 8) hipLaunchKernelGGL((k_gemv_stream<MB, 8>), grid, dim3(64 * 8), 0, s, g);
	else hipLaunchKernelGGL((k_gemv_stream<MB, 4>), grid, dim3(64 * 4), 0, s, g);
}

void gemm(const GemmArgs& g, hipStream_t s) {
	if (g.M <= 0 || g.N <= 0) return;
	if (g.M <= 64 && g.K % 128 == 0) {
		// enough waves to cover the chip: few output tiles -> more waves per tile along K
		const int tiles = (g.N + 15) / 16;
		int waves = tiles >= 1024 ? 4 : (tiles >= 256 ? 8 : 16);
		const int mblocks = (g.M + 15) / 16;
		if (mblocks >= 3 && waves > 8) waves = 8;
		switch (mblocks) {
			case 1: launch_gemv<1>(g, waves, s); break;
			case 2: launch_gemv<2>(g, waves, s); break;
			case 3: launch_gemv<3>(g, waves, s); break;
			default: launch_gemv<4>(g, waves, s); break;
		}
		return;
	}
	dim3 grid((g.N + kBN - 1) / kBN, (g.M + kBM - 1) / kBM);
	hipLaunchKernelGGL(k_gemm_tiled, grid, dim3(kBlock), 0, s, g);
}

void embed(const int32_t* tokens, int M, const int8_t* embed_w, int H, int vocab, Scale site, int8_t* out_codes,
           const int32_t* out_idx, Scale* out_scale, const int32_t* scale_idx, const TokenInfo* tok,
           int32_t* status, hipStream_t s) {
	hipLaunchKernelGGL(k_embed, dim3(M), dim3(kRowBlock), 0, s, tokens, embed_w, H, vocab, site, out_codes, out_idx,
	                   out_scale, scale_idx, tok, status);
}

void rmsnorm(const RowNormArgs& a, int M, int H, const TokenInfo* tok, int32_t* status, int32_t layer,
             hipStream_t s) {
	hipLaunchKernelGGL(k_rmsnorm, dim3(M), dim3(kRowBlock), 0, s, a, H, tok, status, layer);
}

void qkv_post(const QkvPostArgs& a, hipStream_t s) {
	hipLaunchKernelGGL(k_qkv_post, dim3(a.M), dim3(kRowBlock), 0, s, a);
}

void attention(const AttnArgs& a, hipStream_t s) {
	const int group = a.NH / a.NKV;
	const size_t lds = (size_t)group * a.cap * sizeof(int64_t);
	const int use_lds = lds <= 48 * 1024 ? 1 : 0;
	hipLaunchKernelGGL(k_attention, dim3(a.NKV, a.M), dim3(kBlock), use_lds ? lds : 0, s, a, use_lds);
}

void funnel(const FunnelArgs& a, hipStream_t s) { hipLaunchKernelGGL(k_funnel, dim3(a.M), dim3(kRowBlock), 0, s, a); }

void residual_norm(const ResidualArgs& a, hipStream_t s) {
	hipLaunchKernelGGL(k_residual_norm, dim3(a.M), dim3(kRowBlock), 0, s, a);
}

void mlp_act(const ActArgs& a, hipStream_t s) { hipLaunchKernelGGL(k_mlp_act, dim3(a.M), dim3(kRowBlock), 0, s, a); }

void lora_u(const LoraUArgs& a, hipStream_t s) { hipLaunchKernelGGL(k_lora_u, dim3(a.M), dim3(kBlock), 0, s, a); }

void argmax_finalize(const unsigned long long* keys, int ntiles, int M, int32_t* out_tokens, hipStream_t s) {
	hipLaunchKernelGGL(k_argmax_finalize, dim3(M), dim3(kBlock), 0, s, keys, ntiles, out_tokens);
}

}  // namespace sslm_launch
