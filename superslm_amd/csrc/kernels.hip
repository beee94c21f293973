// HIP kernels of the SuperSLM integer forward path for gfx950 (CDNA4).
//
// Every kernel computes exactly what the reference CPU path computes (src/matmul.cpp,
// src/intmath.cpp, src/silu_lut.cpp, src/forward/*.cpp); integer sums are order-free, so tiling,
// split-K and wavefront reductions change no bit.  Rejections are reported per sequence slot in a
// status word instead of aborting (the reference's SslmForwardStatus values).
#include <hip/hip_runtime.h>

#include "kernels.h"

namespace sslm {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kBlock = 256;

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

// block-wide reductions over kBlock threads; `red` holds kBlock/64 slots
__device__ __forceinline__ uint64_t block_max_u64(uint64_t v, uint64_t* red) {
	v = wave_max_u64(v);
	const int w = threadIdx.x >> 6;
	__syncthreads();
	if ((threadIdx.x & 63) == 0) red[w] = v;
	__syncthreads();
	uint64_t r = red[0];
	for (int i = 1; i < kBlock / 64; ++i) r = red[i] > r ? red[i] : r;
	return r;
}

__device__ __forceinline__ int64_t block_sum_i64(int64_t v, int64_t* red) {
	v = wave_sum_i64(v);
	const int w = threadIdx.x >> 6;
	__syncthreads();
	if ((threadIdx.x & 63) == 0) red[w] = v;
	__syncthreads();
	int64_t r = 0;
	for (int i = 0; i < kBlock / 64; ++i) r += red[i];
	return r;
}

__device__ __forceinline__ int64_t block_max_i64(int64_t v, int64_t* red) {
	v = wave_max_i64(v);
	const int w = threadIdx.x >> 6;
	__syncthreads();
	if ((threadIdx.x & 63) == 0) red[w] = v;
	__syncthreads();
	int64_t r = red[0];
	for (int i = 1; i < kBlock / 64; ++i) r = red[i] > r ? red[i] : r;
	return r;
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

// ------------------------------------------------------------------------------------------
// skinny MFMA GEMM for decode (M <= 16*MB per launch row-block): D[t][j] = sum_k x[t][k] w[j][k]
// One wave owns 16 output channels; v_mfma_i32_16x16x64_i8 with tokens as the 16-row operand.
// Split-K partials go through int32 atomics and the last-arriving block runs the epilogue.
// ------------------------------------------------------------------------------------------
__device__ __forceinline__ v4i load16(const int8_t* p) { return *(const v4i*)p; }

template <int MB>
__global__ __launch_bounds__(kBlock) void k_gemv(GemmArgs g) {
	const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
	const int col0 = (blockIdx.x * 4 + wave) * 16;
	const int t_base = blockIdx.z * 16 * MB;
	const int k_begin = blockIdx.y * g.k_split;
	const int k_end = min(g.K, k_begin + g.k_split);
	const int kofs = (lane >> 4) * 16;
	const int my_col = col0 + (lane & 15);
	v4i acc[MB];
#pragma unroll
	for (int mb = 0; mb < MB; ++mb) acc[mb] = v4i{0, 0, 0, 0};
	const bool col_ok = my_col < g.N;
	const int8_t* wrow = g.w + (size_t)(col_ok ? my_col : 0) * g.K;
	for (int k = k_begin; k < k_end; k += 64) {
		const bool kok = k + kofs < k_end;
		v4i b = (col_ok && kok) ? load16(wrow + k + kofs) : v4i{0, 0, 0, 0};
#pragma unroll
		for (int mb = 0; mb < MB; ++mb) {
			const int row = t_base + mb * 16 + (lane & 15);
			v4i a = (row < g.M && kok) ? load16(g.a + (size_t)row * g.lda + k + kofs) : v4i{0, 0, 0, 0};
			acc[mb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc[mb], 0, 0, 0);
		}
	}
	const Epilogue& e = g.epi;
	if (gridDim.y == 1) {
		// direct epilogue: lane holds channel col0 + lane%16, tokens 4*(lane/16) + v
#pragma unroll
		for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
			for (int v = 0; v < 4; ++v) {
				const int t = t_base + mb * 16 + (lane >> 4) * 4 + v;
				const int j = col0 + (lane & 15);
				uint64_t key = 0;
				uint32_t mabs = 0;
				int seg = 0;
				bool live = t < g.M && j < g.N;
				if (live) {
					if (e.raw_out) {
						e.raw_out[(size_t)t * g.N + j] = acc[mb][v];
					} else if (e.argmax_key) {
						const uint32_t logit = (uint32_t)acc[mb][v] ^ 0x80000000u;
						key = ((uint64_t)logit << 32) | (uint64_t)(0xffffffffu - (uint32_t)j);
					} else {
						EpiResult r = epi_value(e, t, j, acc[mb][v]);
						if (!r.ok) set_status(e.status, e.tok[t].slot, e.layer, kBiasReconcileProductOutOfDomain);
						epi_store(e, r, t, j);
						seg = r.seg;
						if (e.seg[r.seg].mode == kSegFunnel) mabs = sat_abs_u32(r.v);
					}
				}
				// reduce across the 16 lanes sharing token t (and the segment is uniform per
				// 16-column wave tile as long as segment bounds are multiples of 16)
				for (int o = 8; o > 0; o >>= 1) {
					uint64_t ok2 = __shfl_xor(key, o, 16);
					key = ok2 > key ? ok2 : key;
					uint32_t om = __shfl_xor(mabs, o, 16);
					mabs = om > mabs ? om : mabs;
				}
				if ((lane & 15) == 0 && t < g.M) {
					if (e.argmax_key) {
						if (key) atomicMax(&e.argmax_key[t], (unsigned long long)key);
					} else if (col0 < g.N && e.seg[seg].mode == kSegFunnel && e.seg[seg].maxabs) {
						atomicMax(&e.seg[seg].maxabs[t], mabs);
					}
				}
			}
		}
		return;
	}
	// split-K: accumulate partials
#pragma unroll
	for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
		for (int v = 0; v < 4; ++v) {
			const int t = t_base + mb * 16 + (lane >> 4) * 4 + v;
			const int j = col0 + (lane & 15);
			if (t < g.M && j < g.N) atomicAdd(&g.acc[(size_t)t * g.N + j], acc[mb][v]);
		}
	}
	__threadfence();
	__shared__ uint32_t s_last;
	__syncthreads();
	const int tile = blockIdx.z * gridDim.x + blockIdx.x;
	if (threadIdx.x == 0) {
		uint32_t prev = atomicAdd(&g.tile_cnt[tile], 1u);
		s_last = (prev == gridDim.y - 1) ? 1u : 0u;
	}
	__syncthreads();
	if (!s_last) return;
	__threadfence();
	// last block: the tile is 64 columns x 16*MB tokens; thread -> column tid%64, token rows
	const int j = blockIdx.x * 64 + (threadIdx.x & 63);
	for (int tt = threadIdx.x >> 6; tt < 16 * MB; tt += kBlock / 64) {
		const int t = t_base + tt;
		uint32_t mabs = 0;
		int seg = 0;
		uint64_t key = 0;
		if (t < g.M && j < g.N) {
			const int32_t a = atomicExch(&g.acc[(size_t)t * g.N + j], 0);
			if (e.raw_out) {
				e.raw_out[(size_t)t * g.N + j] = a;
			} else if (e.argmax_key) {
				const uint32_t logit = (uint32_t)a ^ 0x80000000u;
				key = ((uint64_t)logit << 32) | (uint64_t)(0xffffffffu - (uint32_t)j);
			} else {
				EpiResult r = epi_value(e, t, j, a);
				if (!r.ok) set_status(e.status, e.tok[t].slot, e.layer, kBiasReconcileProductOutOfDomain);
				epi_store(e, r, t, j);
				seg = r.seg;
				if (e.seg[r.seg].mode == kSegFunnel) mabs = sat_abs_u32(r.v);
			}
		}
		// a wave covers 64 consecutive columns of one token; segments are multiples of 16 wide
		// so reduce per 16-lane group
		for (int o = 8; o > 0; o >>= 1) {
			uint64_t ok2 = __shfl_xor(key, o, 16);
			key = ok2 > key ? ok2 : key;
			uint32_t om = __shfl_xor(mabs, o, 16);
			mabs = om > mabs ? om : mabs;
		}
		if ((threadIdx.x & 15) == 0 && t < g.M && j < g.N) {
			if (e.argmax_key) {
				atomicMax(&e.argmax_key[t], (unsigned long long)key);
			} else if (e.seg[seg].mode == kSegFunnel && e.seg[seg].maxabs) {
				atomicMax(&e.seg[seg].maxabs[t], mabs);
			}
		}
	}
	if (threadIdx.x == 0) g.tile_cnt[tile] = 0;
}

// ------------------------------------------------------------------------------------------
// tiled MFMA GEMM for prefill chunks: 128x128 block tile, BK=64, LDS-staged A and B,
// v_mfma_i32_32x32x32_i8, each wave a 64x64 sub-tile (2x2 MFMA tiles).
// ------------------------------------------------------------------------------------------
constexpr int kBM = 128, kBN = 128, kBK = 64, kLdsStride = 80;  // padded row stride (bytes)

__global__ __launch_bounds__(kBlock) void k_gemm_tiled(GemmArgs g) {
	__shared__ __attribute__((aligned(16))) int8_t sa[2][kBM * kLdsStride];
	__shared__ __attribute__((aligned(16))) int8_t sb[2][kBN * kLdsStride];
	const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
	const int m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;
	const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
	v16i acc[2][2];
#pragma unroll
	for (int i = 0; i < 2; ++i)
#pragma unroll
		for (int j = 0; j < 2; ++j)
			for (int v = 0; v < 16; ++v) acc[i][j][v] = 0;

	// global->LDS: each thread moves 2x16B of A and 2x16B of B per K step
	// tile 128 rows x 64 bytes = 512 chunks of 16B; thread t handles chunks t and t+256
	auto gload = [&](int k0, v4i ra[2], v4i rb[2]) {
#pragma unroll
		for (int c = 0; c < 2; ++c) {
			const int chunk = threadIdx.x + c * kBlock;
			const int r = chunk >> 2, kc = (chunk & 3) * 16;
			const int gm = m0 + r, gn = n0 + r;
			const bool kok = k0 + kc < g.K;
			ra[c] = (gm < g.M && kok) ? load16(g.a + (size_t)gm * g.lda + k0 + kc) : v4i{0, 0, 0, 0};
			rb[c] = (gn < g.N && kok) ? load16(g.w + (size_t)gn * g.K + k0 + kc) : v4i{0, 0, 0, 0};
		}
	};
	auto sstore = [&](int buf, const v4i ra[2], const v4i rb[2]) {
#pragma unroll
		for (int c = 0; c < 2; ++c) {
			const int chunk = threadIdx.x + c * kBlock;
			const int r = chunk >> 2, kc = (chunk & 3) * 16;
			*(v4i*)&sa[buf][r * kLdsStride + kc] = ra[c];
			*(v4i*)&sb[buf][r * kLdsStride + kc] = rb[c];
		}
	};
	v4i ra[2], rb[2];
	gload(0, ra, rb);
	sstore(0, ra, rb);
	__syncthreads();
	const int nk = (g.K + kBK - 1) / kBK;
	for (int it = 0; it < nk; ++it) {
		const int buf = it & 1;
		if (it + 1 < nk) gload((it + 1) * kBK, ra, rb);
#pragma unroll
		for (int ks = 0; ks < 2; ++ks) {  // two K=32 MFMA steps per BK=64
			const int kk = ks * 32 + (lane >> 5) * 16;
			v4i af[2], bf[2];
#pragma unroll
			for (int i = 0; i < 2; ++i) af[i] = *(const v4i*)&sa[buf][(wm + i * 32 + (lane & 31)) * kLdsStride + kk];
#pragma unroll
			for (int j = 0; j < 2; ++j) bf[j] = *(const v4i*)&sb[buf][(wn + j * 32 + (lane & 31)) * kLdsStride + kk];
#pragma unroll
			for (int i = 0; i < 2; ++i)
#pragma unroll
				for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
		}
		if (it + 1 < nk) {
			__syncthreads();
			sstore(buf ^ 1, ra, rb);
			__syncthreads();
		}
	}
	// epilogue: 32x32 output layout -- lane holds column lane%32, rows 8*(v/4) + 4*(lane/32) + v%4
	const Epilogue& e = g.epi;
#pragma unroll
	for (int i = 0; i < 2; ++i) {
#pragma unroll
		for (int j = 0; j < 2; ++j) {
#pragma unroll
			for (int v = 0; v < 16; ++v) {
				const int t = m0 + wm + i * 32 + (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3);
				const int col = n0 + wn + j * 32 + (lane & 31);
				uint32_t mabs = 0;
				int seg = 0;
				uint64_t key = 0;
				if (t < g.M && col < g.N) {
					if (e.raw_out) {
						e.raw_out[(size_t)t * g.N + col] = acc[i][j][v];
					} else if (e.argmax_key) {
						const uint32_t logit = (uint32_t)acc[i][j][v] ^ 0x80000000u;
						key = ((uint64_t)logit << 32) | (uint64_t)(0xffffffffu - (uint32_t)col);
					} else {
						EpiResult r = epi_value(e, t, col, acc[i][j][v]);
						if (!r.ok) set_status(e.status, e.tok[t].slot, e.layer, kBiasReconcileProductOutOfDomain);
						epi_store(e, r, t, col);
						seg = r.seg;
						if (e.seg[r.seg].mode == kSegFunnel) mabs = sat_abs_u32(r.v);
					}
				}
				for (int o = 8; o > 0; o >>= 1) {  // 16-lane groups share a token and a segment
					uint64_t ok2 = __shfl_xor(key, o, 16);
					key = ok2 > key ? ok2 : key;
					uint32_t om = __shfl_xor(mabs, o, 16);
					mabs = om > mabs ? om : mabs;
				}
				if ((lane & 15) == 0 && t < g.M && col < g.N) {
					if (e.argmax_key) {
						atomicMax(&e.argmax_key[t], (unsigned long long)key);
					} else if (e.seg[seg].mode == kSegFunnel && e.seg[seg].maxabs) {
						atomicMax(&e.seg[seg].maxabs[t], mabs);
					}
				}
			}
		}
	}
}

// ------------------------------------------------------------------------------------------
// row kernels (one 256-thread block per token)
// ------------------------------------------------------------------------------------------

// forward_sites.cpp:763-787 -- embed row -> funnel ("embed" site, empty incoming)
__global__ __launch_bounds__(kBlock) void k_embed(const int32_t* tokens, const int8_t* embed_w, int H, int vocab,
                                                  Scale site, int8_t* out_codes, const int32_t* out_idx,
                                                  Scale* out_scale, const int32_t* scale_idx, const TokenInfo* tok,
                                                  int32_t* status) {
	__shared__ uint64_t red[kBlock / 64];
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
	for (int i = threadIdx.x; i < H; i += kBlock) {
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
	for (int i = threadIdx.x; i < H; i += kBlock) out[i] = requant_code_small(row[i], (uint64_t)plan.r, plan.s);
	if (threadIdx.x == 0) out_scale[scale_idx[t]] = plan.out;
}

// forward_sites.cpp:410-459 -- the RMSNorm site body, shared by the fused row kernels.
// Writes codes to `out` (row of the current token) and returns the status.
__device__ int32_t rmsnorm_row(const int8_t* h, const int32_t* g, int H, Scale site, int8_t* out, Scale* out_scale,
                               int64_t* out_recip, uint64_t* red_u, int64_t* red_s) {
	__shared__ int64_t s_root;
	__shared__ FunnelPlan plan;
	__shared__ int32_t st;
	int64_t ss = 0;
	for (int i = threadIdx.x; i < H; i += kBlock) ss += (int64_t)h[i] * h[i];
	ss = block_sum_i64(ss, red_s);
	if (threadIdx.x == 0) {
		int64_t root = isqrt(floor_div(ss << 32, (int64_t)H));
		s_root = root > 1 ? root : 1;
	}
	__syncthreads();
	const int64_t root = s_root;
	uint64_t mx = 0;
	for (int i = threadIdx.x; i < H; i += kBlock) {
		int64_t w = floor_div((int64_t)h[i] << 32, root) * (int64_t)g[i];
		uint64_t a = w < 0 ? (uint64_t)0 - (uint64_t)w : (uint64_t)w;
		mx = a > mx ? a : mx;
	}
	mx = block_max_u64(mx, red_u);
	if (threadIdx.x == 0) st = funnel_plan(mx, nullptr, 0, site, &plan);
	__syncthreads();
	if (st != kOk) return st;
	for (int i = threadIdx.x; i < H; i += kBlock) {
		int64_t w = floor_div((int64_t)h[i] << 32, root) * (int64_t)g[i];
		out[i] = requant_code_small(w, (uint64_t)plan.r, plan.s);
	}
	if (threadIdx.x == 0) {
		*out_scale = plan.out;
		if (out_recip) *out_recip = fits_i32(plan.out.m) ? reciprocal(plan.out.m) : 0;
	}
	__syncthreads();
	return kOk;
}

__global__ __launch_bounds__(kBlock) void k_rmsnorm(sslm_launch::RowNormArgs a, int H, const TokenInfo* tok,
                                                    int32_t* status, int32_t layer) {
	__shared__ uint64_t red_u[kBlock / 64];
	__shared__ int64_t red_s[kBlock / 64];
	const int t = blockIdx.x;
	if (status[tok[t].slot] != 0) return;
	const int8_t* h = a.in_codes + (size_t)a.in_idx[t] * a.ld_in;
	int32_t st = rmsnorm_row(h, a.gain, H, a.site, a.out + (size_t)t * H, &a.out_scale[t],
	                         a.out_recip ? &a.out_recip[t] : nullptr, red_u, red_s);
	if (threadIdx.x == 0) set_status(status, tok[t].slot, layer, st);
}

// q funnel + RoPE(q); K/V landing, RoPE(K), KV write (forward_sites.cpp:1281-1418, :1748-1787)
__global__ __launch_bounds__(kBlock) void k_qkv_post(sslm_launch::QkvPostArgs a) {
	__shared__ FunnelPlan plan;
	__shared__ int32_t st;
	__shared__ unsigned long long sat_block;
	const int t = blockIdx.x;
	const TokenInfo ti = a.tok[t];
	if (a.status[ti.slot] != 0) return;
	const int H = a.H, D = a.D, pairs = D / 2;
	const int64_t pos = ti.pos;
	if (threadIdx.x == 0) {
		sat_block = 0;
		const Scale inc = a.in_scale[t];
		uint32_t mx = a.q_maxabs[t];
		a.q_maxabs[t] = 0;
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
	for (int p = threadIdx.x; p < H / 2; p += kBlock) {
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
	for (int p = threadIdx.x; p < KVH / 2; p += kBlock) {
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
			sc[(int64_t)g * a.cap + p] = (e << 15) / denom;
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
	if (threadIdx.x == 0) atomicMax(&a.ctx_maxabs[t], mabs > 0xffffffffull ? 0xffffffffu : (uint32_t)mabs);
}

// funnel over an int32 fold-output row (checked_chain_funnel.cpp:257-364)
__global__ __launch_bounds__(kBlock) void k_funnel(sslm_launch::FunnelArgs a) {
	__shared__ FunnelPlan plan;
	__shared__ int32_t st;
	const int t = blockIdx.x;
	const int slot = a.tok[t].slot;
	if (a.status[slot] != 0) {
		if (threadIdx.x == 0) a.maxabs[t] = 0;
		return;
	}
	if (threadIdx.x == 0) {
		uint32_t mx = a.maxabs[t];
		a.maxabs[t] = 0;
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
	for (int i = threadIdx.x; i < a.N; i += kBlock) a.out[(size_t)t * a.N + i] = requant_code_small(f[i], (uint64_t)plan.r, plan.s);
	if (threadIdx.x == 0) a.out_scale[t] = plan.out;
}

// projection funnel -> residual reconcile -> (optional) RMSNorm, all on one token's row
// (forward_sites.cpp:871-989 residual; :410-459 norm)
__global__ __launch_bounds__(kBlock) void k_residual_norm(sslm_launch::ResidualArgs a) {
	__shared__ FunnelPlan bplan, rplan;
	__shared__ int32_t st;
	__shared__ int64_t r_h;
	__shared__ uint64_t red_u[kBlock / 64];
	__shared__ int64_t red_s[kBlock / 64];
	const int t = blockIdx.x;
	const int slot = a.tok[t].slot;
	const int H = a.H;
	if (a.status[slot] != 0) {
		if (threadIdx.x == 0) a.branch_maxabs[t] = 0;
		return;
	}
	const int8_t* stream = a.stream + (size_t)a.stream_idx[t] * H;
	const Scale ss = a.stream_scale[a.stream_idx[t]];
	if (threadIdx.x == 0) {
		uint32_t mx = a.branch_maxabs[t];
		a.branch_maxabs[t] = 0;
		const Scale inc = a.branch_in[t];
		st = funnel_plan(mx, &inc, 1, a.branch_site, &bplan);
		if (st == kOk && !fits_i32(ss.m)) st = kCarriedScaleMantissaOutOfDomain;
		if (st == kOk) r_h = reciprocal(ss.m);
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
	for (int i = threadIdx.x; i < H; i += kBlock) {
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
	for (int i = threadIdx.x; i < H; i += kBlock) {
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
__global__ __launch_bounds__(kBlock) void k_mlp_act(sslm_launch::ActArgs a) {
	__shared__ FunnelPlan gp, up, ap;
	__shared__ int32_t st;
	__shared__ uint64_t red_u[kBlock / 64];
	const int t = blockIdx.x;
	const int slot = a.tok[t].slot;
	const int I = a.I;
	if (a.status[slot] != 0) {
		if (threadIdx.x == 0) {
			a.gate_maxabs[t] = 0;
			a.up_maxabs[t] = 0;
		}
		return;
	}
	if (threadIdx.x == 0) {
		const Scale inc = a.in_scale[t];
		uint32_t gm = a.gate_maxabs[t], um = a.up_maxabs[t];
		a.gate_maxabs[t] = 0;
		a.up_maxabs[t] = 0;
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
	for (int i = threadIdx.x; i < I; i += kBlock) {
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
	for (int i = threadIdx.x; i < I; i += kBlock) {
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

__global__ void k_argmax_finalize(unsigned long long* keys, int M, int32_t* out) {
	const int t = blockIdx.x * blockDim.x + threadIdx.x;
	if (t >= M) return;
	const unsigned long long k = keys[t];
	out[t] = (int32_t)(0xffffffffu - (uint32_t)(k & 0xffffffffull));
	keys[t] = 0;
}

}  // namespace sslm

// ------------------------------------------------------------------------------------------
// launch wrappers
// ------------------------------------------------------------------------------------------
namespace sslm_launch {

void gemm(const GemmArgs& g, hipStream_t s) {
	if (g.M <= 0 || g.N <= 0) return;
	if (g.M > 64) {
		dim3 grid((g.N + kBN - 1) / kBN, (g.M + kBM - 1) / kBM);
		hipLaunchKernelGGL(k_gemm_tiled, grid, dim3(kBlock), 0, s, g);
		return;
	}
	const int splits = (g.K + g.k_split - 1) / g.k_split;
	const int mblocks = (g.M + 15) / 16;
	dim3 grid((g.N + 63) / 64, splits, 1);
	switch (mblocks) {
		case 1: hipLaunchKernelGGL(k_gemv<1>, grid, dim3(kBlock), 0, s, g); break;
		case 2: hipLaunchKernelGGL(k_gemv<2>, grid, dim3(kBlock), 0, s, g); break;
		case 3: hipLaunchKernelGGL(k_gemv<3>, grid, dim3(kBlock), 0, s, g); break;
		default: hipLaunchKernelGGL(k_gemv<4>, grid, dim3(kBlock), 0, s, g); break;
	}
}

void embed(const int32_t* tokens, int M, const int8_t* embed_w, int H, int vocab, Scale site, int8_t* out_codes,
           const int32_t* out_idx, Scale* out_scale, const int32_t* scale_idx, const TokenInfo* tok,
           int32_t* status, hipStream_t s) {
	hipLaunchKernelGGL(k_embed, dim3(M), dim3(kBlock), 0, s, tokens, embed_w, H, vocab, site, out_codes, out_idx,
	                   out_scale, scale_idx, tok, status);
}

void rmsnorm(const RowNormArgs& a, int M, int H, const TokenInfo* tok, int32_t* status, int32_t layer,
             hipStream_t s) {
	hipLaunchKernelGGL(k_rmsnorm, dim3(M), dim3(kBlock), 0, s, a, H, tok, status, layer);
}

void qkv_post(const QkvPostArgs& a, hipStream_t s) {
	hipLaunchKernelGGL(k_qkv_post, dim3(a.M), dim3(kBlock), 0, s, a);
}

void attention(const AttnArgs& a, hipStream_t s) {
	const int group = a.NH / a.NKV;
	const size_t lds = (size_t)group * a.cap * sizeof(int64_t);
	const int use_lds = lds <= 48 * 1024 ? 1 : 0;
	hipLaunchKernelGGL(k_attention, dim3(a.NKV, a.M), dim3(kBlock), use_lds ? lds : 0, s, a, use_lds);
}

void funnel(const FunnelArgs& a, hipStream_t s) { hipLaunchKernelGGL(k_funnel, dim3(a.M), dim3(kBlock), 0, s, a); }

void residual_norm(const ResidualArgs& a, hipStream_t s) {
	hipLaunchKernelGGL(k_residual_norm, dim3(a.M), dim3(kBlock), 0, s, a);
}

void mlp_act(const ActArgs& a, hipStream_t s) { hipLaunchKernelGGL(k_mlp_act, dim3(a.M), dim3(kBlock), 0, s, a); }

void lora_u(const LoraUArgs& a, hipStream_t s) { hipLaunchKernelGGL(k_lora_u, dim3(a.M), dim3(kBlock), 0, s, a); }

void argmax_finalize(unsigned long long* keys, int M, int32_t* out_tokens, hipStream_t s) {
	hipLaunchKernelGGL(k_argmax_finalize, dim3((M + 63) / 64), dim3(64), 0, s, keys, M, out_tokens);
}

}  // namespace sslm_launch
