// HIP kernels of the SuperSLM integer forward path for gfx950 (CDNA4).
//
// Every kernel computes exactly what the reference CPU path computes (src/matmul.cpp,
// src/intmath.cpp, src/silu_lut.cpp, src/forward/*.cpp); integer sums are order-free, so tiling,
// split-K and wavefront reductions change no bit.  Rejections are reported per sequence slot in a
// status word instead of aborting (the reference's SslmForwardStatus values).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>

#include "kernels.h"

// Optional phase timestamps for latency studies of the row kernels; compiled out by default.
#ifndef KT
#define KT(i)
#endif

namespace sslm {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
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

// Row maxima travel as 32-bit magnitudes: |v| saturated at 2^32 - 2, so that 2^32 - 1 (kBad32)
// is free to mark a refusal somewhere in the row.  Every consumer rejects a maximum above 2^31
// (the funnel's accepted domain), so the saturation changes no outcome.
constexpr uint32_t kBad32 = 0xffffffffu;

__device__ __forceinline__ uint32_t sat_abs_u32(int64_t v) {
	uint64_t a = v < 0 ? (uint64_t)0 - (uint64_t)v : (uint64_t)v;
	return a > 0xfffffffeull ? 0xfffffffeu : (uint32_t)a;
}

// The row of a one-block-per-row launch: workgroups go to the 8 XCDs in turn (block b on XCD
// b % 8), so giving each XCD a contiguous run of rows keeps a tile-major maxima array's lines
// ([tile][row], 32 rows to a line) in one XCD's L2 instead of fetched by all eight.  Identity
// when the row count is not a multiple of 8.
__device__ __forceinline__ int xcd_row(int b, int n) { return (n & 7) ? b : (b & 7) * (n >> 3) + (b >> 3); }

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

// LoRA delta of channel jj for token t (forward_sites.cpp:1051-1112): the adapter's B row
// against the token's intermediate codes, amplified by the delta fold.  |B.u| <= 127^2 * rank
// < 2^31, so packed int8 dot products (sdot4) accumulate it exactly in int32; a rank that is not
// a multiple of 4 takes the byte loop out of line.  Plain values only: a reference into the
// kernel arguments would make the compiler copy them to scratch memory.
__device__ __attribute__((noinline)) int32_t lora_dot_bytes(const int8_t* br, const int8_t* ur, int rank) {
	int32_t d = 0;
	for (int r = 0; r < rank; ++r) d += (int32_t)br[r] * (int32_t)ur[r];
	return d;
}

__device__ __forceinline__ int64_t lora_delta_v(const int8_t* lora_b, const int8_t* lora_u, const int32_t* dfold,
                                                int rank, int t, int jj) {
	const int8_t* br = lora_b + (size_t)jj * rank;
	const int8_t* ur = lora_u + (size_t)t * kMaxRank;
	int32_t d = 0;
	if ((rank & 3) == 0) {
		for (int r = 0; r < rank; r += 4)
			d = __builtin_amdgcn_sdot4(*(const int32_t*)(br + r), *(const int32_t*)(ur + r), d, false);
	} else {
		d = lora_dot_bytes(br, ur, rank);
	}
	const int32_t* df = dfold + 3 * jj;
	return apply_amp_fold((int64_t)d, df[0], df[1], df[2]);
}

// Called out of line: adapters are optional, and inlined into an epilogue the delta costs the
// common path registers (the decode GEMV must stay within 128 VGPRs for 4 waves per SIMD) and,
// unrolled per element, code size in the row kernels.
// A leaf function (its byte loop inline, no further call): a non-leaf callee saves its return
// address in scratch memory, and any private segment on a kernel costs every dispatch of it
// about 0.5 us of launch time on MI355X, taken or not.
__device__ __attribute__((noinline)) int64_t lora_delta_cold(const int8_t* lora_b, const int8_t* lora_u,
                                                             const int32_t* dfold, int rank, int t, int jj) {
	const int8_t* br = lora_b + (size_t)jj * rank;
	const int8_t* ur = lora_u + (size_t)t * kMaxRank;
	int32_t d = 0;
	if ((rank & 3) == 0) {
		for (int r = 0; r < rank; r += 4)
			d = __builtin_amdgcn_sdot4(*(const int32_t*)(br + r), *(const int32_t*)(ur + r), d, false);
	} else {
		for (int r = 0; r < rank; ++r) d += (int32_t)br[r] * (int32_t)ur[r];
	}
	const int32_t* df = dfold + 3 * jj;
	return apply_amp_fold((int64_t)d, df[0], df[1], df[2]);
}

__device__ __forceinline__ int64_t lora_delta(const Segment& sg, int rank, int t, int jj) {
	return lora_delta_cold(sg.lora_b, sg.lora_u, sg.lora_dfold, rank, t, jj);
}

__device__ __forceinline__ EpiResult epi_value(const Epilogue& e, int t, int j, int32_t acc) {
	int si = 0;
	while (si + 1 < e.nseg && j >= e.seg[si].n_end) ++si;
	const Segment& sg = e.seg[si];
	const int jj = j - sg.n_begin;
	const int32_t* f = sg.fold + 3 * jj;
	int64_t v = apply_fold((int64_t)acc, f[0], f[1], f[2]);
	if (sg.lora_b) {
		v += lora_delta(sg, e.rank, t, jj);
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
		const uint8_t* pg = e.mask_page ? e.mask_page[t] : nullptr;
		const int32_t v = pg && !((pg[j >> 3] >> (j & 7)) & 1u) ? INT32_MIN : acc;
		const uint32_t logit = (uint32_t)v ^ 0x80000000u;
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
			e.argmax_key[(size_t)t * e.key_ld + tile] = key;
		} else if (!e.raw_out && e.seg[seg].mode == kSegFunnel && e.seg[seg].maxpart) {
			e.seg[seg].maxpart[(size_t)tile * kPartLd + t] = mabs;
		}
	}
}

// ------------------------------------------------------------------------------------------
// Decode GEMV (M <= 64).  A decode projection streams each weight byte once and lasts a few
// microseconds, so the kernel puts as much of the matrix in flight as it can: a block of 4 waves
// owns TPW 16-column tiles and a range of K (split-K over gridDim.y), and each wave issues the
// loads of CPW 128-byte chunks of all its tiles before the MFMAs that consume them.  Per chunk a
// lane holds 32 contiguous bytes of one weight row (a wave covers 16 rows x 128 B per tile) and
// the activations in the same lane->k mapping -- reused across the TPW tiles -- feeding two
// v_mfma_i32_16x16x64_i8 per tile; the k permutation is identical on both operands, so the
// integer sum is exact.  The waves' tiles meet in LDS.  With one split the block runs the
// epilogue; with several, each split stores its raw partial plane and the consumer adds them
// (no cross-block synchronisation inside the kernel).
// ------------------------------------------------------------------------------------------
__device__ __forceinline__ uint32_t dpp_max16(uint32_t v) {
	// row_ror:8, 4, 2, 1 -- every lane of the 16-lane row ends with the row maximum
	uint32_t w = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xf, 0xf, false);
	v = w > v ? w : v;
	w = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x124, 0xf, 0xf, false);
	v = w > v ? w : v;
	w = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x122, 0xf, 0xf, false);
	v = w > v ? w : v;
	w = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x121, 0xf, 0xf, false);
	return w > v ? w : v;
}

// Refused bias reconciles in the decode GEMV epilogue (rare; out of line): bit v of `mask` marks
// token t0 + v.
__device__ __attribute__((noinline)) void set_status_rows(int32_t* status, const TokenInfo* tok, int32_t layer, int t0,
                                                         uint32_t mask) {
	for (int v = 0; v < 4; ++v)
		if (mask >> v & 1) set_status(status, tok[t0 + v].slot, layer, kBiasReconcileProductOutOfDomain);
}

// The fields of segment `si` (wave-uniform) that the decode GEMV epilogue uses, selected with
// constant indices so they stay scalar kernel-argument loads.
struct SegView {
	int32_t n_begin, mode, ld_out;
	void* out;
	uint32_t* maxpart;
	const int32_t* fold;
	const int64_t* bias;
	const int8_t* lora_b;
	const int32_t* lora_dfold;
	const int8_t* lora_u;
};

__device__ __forceinline__ SegView seg_view(const Epilogue& e, int si) {
	const Segment& s = si == 0 ? e.seg[0] : (si == 1 ? e.seg[1] : e.seg[2]);
	return SegView{s.n_begin, s.mode, s.ld_out, s.out, s.maxpart, s.fold, s.bias, s.lora_b, s.lora_dfold, s.lora_u};
}

constexpr int kGemvWaves = 4;

template <int MB, int TPW, int CPW>
__global__ __launch_bounds__(64 * kGemvWaves) void k_gemv(GemmArgs g, int cps) {
	__shared__ v4i red[kGemvWaves][MB * TPW][64];
	const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
	const int tile0 = blockIdx.x * TPW, split = blockIdx.y;
	const int ri = lane & 15, grp = lane >> 4;
	const int C = g.K >> 7;
	const int c_begin = split * cps;
	const int c_end = min(C, c_begin + cps);
	const v4i z = v4i{0, 0, 0, 0};
	const int8_t* wrow[TPW];
	bool col_ok[TPW];
#pragma unroll
	for (int tt = 0; tt < TPW; ++tt) {
		const int col = (tile0 + tt) * 16 + ri;
		col_ok[tt] = col < g.N;
		wrow[tt] = g.w + (size_t)(col_ok[tt] ? col : g.N - 1) * g.K + grp * 32;
	}
	const int8_t* arow[MB];
	bool row_ok[MB];
#pragma unroll
	for (int mb = 0; mb < MB; ++mb) {
		const int r = mb * 16 + ri;
		row_ok[mb] = r < g.M;
		arow[mb] = g.a + (size_t)(row_ok[mb] ? r : g.M - 1) * g.lda + grp * 32;
	}
	// The projection epilogue's parameters for the tile this wave finishes (MB * TPW <=
	// kGemvWaves: one (mb, tile) per wave) are fetched now, so they arrive with the weights.
	// Segment bounds are multiples of 16, so the segment is uniform over the tile and is chosen
	// with wave-uniform values; the loads are unconditional, from always-valid addresses (the
	// weights stand in for unused values), so no branch join waits on them before the loop.
	const Epilogue& e = g.epi;
	const int o_mine = __builtin_amdgcn_readfirstlane(wave);
	const bool proj = g.splits <= 1 && !e.raw_out && !e.argmax_key && o_mine < MB * TPW;
	int si = 0;
	if (proj) {
		const int jt = (tile0 + o_mine % TPW) * 16;
		while (si + 1 < e.nseg && jt >= e.seg[si].n_end) ++si;
	}
	const SegView sg = seg_view(e, si);
	const bool p_lora = proj && sg.lora_b != nullptr, p_bias = proj && sg.bias != nullptr;
	const int jj0 = min((tile0 + o_mine % TPW) * 16 + ri, g.N - 1) - (proj ? sg.n_begin : 0);
	const int32_t* fp = proj ? sg.fold + 3 * jj0 : (const int32_t*)g.w;
	const int32_t p_f0 = fp[0], p_f1 = fp[1], p_f2 = fp[2];
	const int64_t p_b = *(p_bias ? sg.bias + jj0 : (const int64_t*)g.w);
	int64_t p_rcp[4], p_ein[4];
#pragma unroll
	for (int v = 0; v < 4; ++v) {
		const int t = min((o_mine / TPW) * 16 + grp * 4 + v, g.M - 1);
		p_rcp[v] = *(p_bias ? e.in_recip + t : (const int64_t*)g.w);
		p_ein[v] = (p_bias ? e.in_scale + t : (const Scale*)g.w)->e;
	}
	v4i acc[MB][TPW];
#pragma unroll
	for (int mb = 0; mb < MB; ++mb)
#pragma unroll
		for (int tt = 0; tt < TPW; ++tt) acc[mb][tt] = z;
	for (int base = c_begin + wave; base < c_end; base += kGemvWaves * CPW) {
		v4i b[CPW][TPW][2], x[CPW][MB][2];
#pragma unroll
		for (int i = 0; i < CPW; ++i) {  // clamped, unconditional loads; out-of-range chunks add 0
			const int c = min(base + i * kGemvWaves, c_end - 1);
#pragma unroll
			for (int tt = 0; tt < TPW; ++tt) {
				b[i][tt][0] = load16(wrow[tt] + (size_t)c * 128);
				b[i][tt][1] = load16(wrow[tt] + (size_t)c * 128 + 16);
			}
#pragma unroll
			for (int mb = 0; mb < MB; ++mb) {
				x[i][mb][0] = load16(arow[mb] + (size_t)c * 128);
				x[i][mb][1] = load16(arow[mb] + (size_t)c * 128 + 16);
			}
		}
#pragma unroll
		for (int i = 0; i < CPW; ++i) {
			const bool ok = base + i * kGemvWaves < c_end;
#pragma unroll
			for (int mb = 0; mb < MB; ++mb) {
				const v4i x0 = ok && row_ok[mb] ? x[i][mb][0] : z, x1 = ok && row_ok[mb] ? x[i][mb][1] : z;
#pragma unroll
				for (int tt = 0; tt < TPW; ++tt) {
					acc[mb][tt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(x0, b[i][tt][0], acc[mb][tt], 0, 0, 0);
					acc[mb][tt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(x1, b[i][tt][1], acc[mb][tt], 0, 0, 0);
				}
			}
		}
	}
#pragma unroll
	for (int mb = 0; mb < MB; ++mb)
#pragma unroll
		for (int tt = 0; tt < TPW; ++tt) red[wave][mb * TPW + tt][lane] = acc[mb][tt];
	// Drain this wave's loads here (a wave that ran the loop has none left; one that ran no
	// chunk still holds its prologue loads).  Without it the wait counts in the epilogue --
	// which on this target also count stores -- are derived from the no-chunk path and end up
	// waiting for the epilogue's own stores to be acknowledged.
	__builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0), expcnt and lgkmcnt unconstrained
	__syncthreads();
	if (o_mine >= MB * TPW) return;
	const int mb = o_mine / TPW, tile = tile0 + o_mine % TPW;
	v4i tot = red[0][o_mine][lane];
#pragma unroll
	for (int w = 1; w < kGemvWaves; ++w) {
		const v4i y = red[w][o_mine][lane];
		tot[0] += y[0];
		tot[1] += y[1];
		tot[2] += y[2];
		tot[3] += y[3];
	}
	const int j = tile * 16 + ri;
	const int t0 = mb * 16 + grp * 4;  // this lane's tokens: t0 .. t0 + 3
	if (g.splits > 1 || e.raw_out) {
		// raw accumulators: a split-K plane, or the whole sum for a consumer that applies the
		// epilogue on the row
		int32_t* dst = g.splits > 1 ? g.split_part + (size_t)split * g.M * g.N : e.raw_out;
#pragma unroll
		for (int v = 0; v < 4; ++v)
			if (t0 + v < g.M && j < g.N) dst[(size_t)(t0 + v) * g.N + j] = tot[v];
	} else if (e.argmax_key) {
		// per (token, 16-column tile) greedy keys: the larger logit, then the smaller index
#pragma unroll
		for (int v = 0; v < 4; ++v) {
			// a schema-masked token's logit counts as INT32_MIN
			const uint8_t* pg = e.mask_page && t0 + v < g.M ? e.mask_page[t0 + v] : nullptr;
			const int32_t lv = pg && j < g.N && !((pg[j >> 3] >> (j & 7)) & 1u) ? INT32_MIN : tot[v];
			uint64_t key = j < g.N ? ((uint64_t)((uint32_t)lv ^ 0x80000000u) << 32) | (0xffffffffu - (uint32_t)j) : 0;
			for (int o = 8; o > 0; o >>= 1) {
				const uint64_t k2 = __shfl_xor(key, o, 16);
				key = k2 > key ? k2 : key;
			}
			if (ri == 0 && t0 + v < g.M && tile * 16 < g.N) e.argmax_key[(size_t)(t0 + v) * e.key_ld + tile] = key;
		}
	} else {
		// projection epilogue (forward_sites.cpp:1114-1141): WSC1 fold -> LoRA delta -> bias
		// reconcile; every value first, then the stores
		const int jj = j - sg.n_begin;
		const int32_t mode = sg.mode;
		int64_t val[4];
		uint32_t mabs[4];
		uint32_t bad = 0;
#pragma unroll
		for (int v = 0; v < 4; ++v) {
			const bool live = t0 + v < g.M && j < g.N;
			val[v] = apply_fold((int64_t)tot[v], p_f0, p_f1, p_f2);
			if (p_lora && live) val[v] += lora_delta_cold(sg.lora_b, sg.lora_u, sg.lora_dfold, e.rank, t0 + v, jj);
			if (p_bias) {
				int64_t term;
				if (bias_term(p_b, p_rcp[v], p_ein[v], val[v], &term)) val[v] += term;
				else bad |= live ? 1u << v : 0u;
			}
			mabs[v] = dpp_max16(live && mode == kSegFunnel ? sat_abs_u32(val[v]) : 0u);  // tile max
		}
#pragma unroll
		for (int v = 0; v < 4; ++v) {
			if (t0 + v < g.M && j < g.N) {
				if (mode == kSegWide) ((int64_t*)sg.out)[(size_t)(t0 + v) * sg.ld_out + jj] = val[v];
				else ((int32_t*)sg.out)[(size_t)(t0 + v) * sg.ld_out + jj] = sat_i32(val[v]);
			}
			if (mode == kSegFunnel && sg.maxpart && ri == 0 && t0 + v < g.M)
				sg.maxpart[(size_t)tile * kPartLd + t0 + v] = mabs[v];
		}
		if (bad) set_status_rows(e.status, e.tok, e.layer, t0, bad);  // refused bias reconciles (values left unbiased)
	}
}

// ------------------------------------------------------------------------------------------
// Decode GEMV, persistent form (M <= 16, K <= 4096), for projection launches whose segments are
// funnel or wide outputs without bias or LoRA (gate|up).  One block per CU walks 16-column
// tiles blockIdx.x, + gridDim.x, ...; wave w keeps its K chunks (w + 4 i) of the 16 activation
// rows in registers for the whole launch and loads the next tile's weight chunks (and fold
// parameters) while it multiplies the current tile's, two register sets alternating; the four
// partial sums meet in a double-buffered LDS slot and every wave applies the epilogue of k_gemv
// (WSC1 fold, 16-lane tile maximum, stores) to a quarter of the tile, one token row of each
// group of four per wave (one wave per tile, rotating, held the other three at the next
// barrier: in-step gate|up 9.9 -> 9.1 us).  Against one block per tile pair, whose load ->
// reduce -> epilogue runs once per block with nothing behind it: gate|up at 16 tokens with
// HBM-cold weights 11.5 -> 9 us.
// ------------------------------------------------------------------------------------------
// segment of the 16-column tile starting at column c0 (bounds are multiples of 16), with
// constant indices so the fields stay scalar kernel-argument loads
__device__ __forceinline__ int tile_segment(const Epilogue& e, int c0) {
	return (e.nseg > 1 && c0 >= e.seg[0].n_end) ? ((e.nseg > 2 && c0 >= e.seg[1].n_end) ? 2 : 1) : 0;
}

template <int MB, int CPW>  // MB row groups of 16 tokens
__global__ __launch_bounds__(256) void k_gemv_p(GemmArgs g) {
	__shared__ v4i red[2][kGemvWaves][MB][64];
	const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, ri = lane & 15, grp = lane >> 4;
	const int C = g.K >> 7, T = (g.N + 15) / 16;
	const v4i z = v4i{0, 0, 0, 0};
	const Epilogue& e = g.epi;
	v4i x[MB][CPW][2];
#pragma unroll
	for (int mb = 0; mb < MB; ++mb) {
		const int r = mb * 16 + ri;
		const bool rok = r < g.M;
		const int8_t* arow = g.a + (size_t)(rok ? r : g.M - 1) * g.lda + grp * 32;
#pragma unroll
		for (int i = 0; i < CPW; ++i) {
			const int c = wave + kGemvWaves * i;
			const bool ok = rok && c < C;
			x[mb][i][0] = ok ? load16(arow + (size_t)c * 128) : z;
			x[mb][i][1] = ok ? load16(arow + (size_t)c * 128 + 16) : z;
		}
	}
	// weight chunks and fold parameters of tile t (past the last tile: the last one again)
	struct Tile {
		v4i b[CPW][2];
		int32_t f0, f1, f2;
	};
	auto load_tile = [&](int t, Tile& d) {
		const int tc = t < T ? t : T - 1;
		const int col = min(tc * 16 + ri, g.N - 1);
		const int8_t* wr = g.w + (size_t)col * g.K + grp * 32;
#pragma unroll
		for (int i = 0; i < CPW; ++i) {
			const int c = min(wave + kGemvWaves * i, C - 1);
			d.b[i][0] = load16(wr + (size_t)c * 128);
			d.b[i][1] = load16(wr + (size_t)c * 128 + 16);
		}
		const int si = tile_segment(e, tc * 16);
		const int32_t* fp = (si == 0 ? e.seg[0].fold : (si == 1 ? e.seg[1].fold : e.seg[2].fold)) +
		                    3 * (col - (si == 0 ? e.seg[0].n_begin : (si == 1 ? e.seg[1].n_begin : e.seg[2].n_begin)));
		d.f0 = fp[0];
		d.f1 = fp[1];
		d.f2 = fp[2];
	};
	auto step = [&](int tile, int it, Tile& cur, Tile& nxt) {
		load_tile(tile + (int)gridDim.x, nxt);
		v4i acc[MB];
#pragma unroll
		for (int mb = 0; mb < MB; ++mb) {
			acc[mb] = z;
#pragma unroll
			for (int i = 0; i < CPW; ++i)
				if (wave + kGemvWaves * i < C) {
					acc[mb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(x[mb][i][0], cur.b[i][0], acc[mb], 0, 0, 0);
					acc[mb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(x[mb][i][1], cur.b[i][1], acc[mb], 0, 0, 0);
				}
			red[it & 1][wave][mb][lane] = acc[mb];
		}
		__syncthreads();
		// every wave takes a quarter of the epilogue: row v = wave of each 4-token group, one value
		// per lane, so no wave carries a whole tile's epilogue into the next tile's barrier
		const SegView sg = seg_view(e, tile_segment(e, tile * 16));
		const int j = tile * 16 + ri, jj = j - sg.n_begin, v = wave;
#pragma unroll
		for (int mb = 0; mb < MB; ++mb) {
			int32_t tot = 0;
#pragma unroll
			for (int w = 0; w < kGemvWaves; ++w) tot += ((const int32_t*)&red[it & 1][w][mb][lane])[v];
			const int tk = mb * 16 + grp * 4 + v;
			const bool live = tk < g.M && j < g.N;
			const int64_t val = apply_fold((int64_t)tot, cur.f0, cur.f1, cur.f2);
			const uint32_t mabs = dpp_max16(live && sg.mode == kSegFunnel ? sat_abs_u32(val) : 0u);  // tile max
			if (live) {
				if (sg.mode == kSegWide) ((int64_t*)sg.out)[(size_t)tk * sg.ld_out + jj] = val;
				else ((int32_t*)sg.out)[(size_t)tk * sg.ld_out + jj] = sat_i32(val);
			}
			if (sg.mode == kSegFunnel && sg.maxpart && ri == 0 && tk < g.M) sg.maxpart[(size_t)tile * kPartLd + tk] = mabs;
		}
	};
	Tile t0buf, t1buf;
	int tile = blockIdx.x, it = 0;
	load_tile(tile, t0buf);
	while (tile < T) {
		step(tile, it, t0buf, t1buf);
		tile += gridDim.x;
		++it;
		if (tile >= T) break;
		step(tile, it, t1buf, t0buf);
		tile += gridDim.x;
		++it;
	}
}

// ------------------------------------------------------------------------------------------
// LM head on the packed decode copy (M <= 32, K <= 4096), persistent: one block per CU walks the
// 16-column tiles blockIdx.x, + gridDim.x, ...; wave w keeps K chunks w CPW .. + CPW of the MB
// 16-token row groups in registers for the whole launch and loads the next tile's weight chunks
// while it multiplies the current tile's, two register sets alternating (the loop body is two
// steps, so the wait counts stay exact).  The four partial sums meet in a double-buffered LDS
// slot; every wave finishes one token row of each 4-token group: the per (token, tile) greedy
// key of k_gemv_w (the larger logit, then the smaller index; a schema-masked token's logit counts
// as INT32_MIN).  Each block reads the activation rows once for all its tiles, where one block
// per tile pair read them once per 32 columns.
// ------------------------------------------------------------------------------------------
__device__ __forceinline__ const int8_t* pk_lane(const int8_t* wp, int tile, int C, int lane);

constexpr int kHeadMaxSteps = 64;  // tiles per block of k_gemv_head (the launch sizes its grid to fit)

template <int MB, int CPW>
__global__ __launch_bounds__(256) void k_gemv_head(GemmArgs g) {
	__shared__ v4i red[2][kGemvWaves][MB][64];
	// the block's keys, stored after the loop: a global store inside it (stores count in the
	// vector-memory counter) left the waits before each step's MFMAs draining the next tile's loads
	__shared__ uint64_t s_key[kHeadMaxSteps][MB * 16];
	const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, ri = lane & 15, grp = lane >> 4;
	const int C = g.K >> 7, T = (g.N + 15) / 16;
	const v4i z = v4i{0, 0, 0, 0};
	const Epilogue& e = g.epi;
	// this lane's epilogue tokens (mb * 16 + 4 grp + wave) and their schema pages: a mask byte
	// travels with each tile's weights, read from a valid address whether or not a page is set, so
	// no wait inside the loop drains the next tile's loads
	const uint8_t* pgp[MB];
	bool masked[MB];
#pragma unroll
	for (int mb = 0; mb < MB; ++mb) {
		const int tk = min(mb * 16 + grp * 4 + wave, g.M - 1);
		const uint8_t* pg = e.mask_page ? e.mask_page[tk] : nullptr;
		masked[mb] = pg != nullptr;
		pgp[mb] = pg ? pg : (const uint8_t*)g.wp;
	}
	struct Tile {
		v4i b[CPW][2];
		uint8_t mbits[MB];
	};
	auto load_tile = [&](int t, Tile& d) {
		const int tc = min(t, T - 1);
		const int8_t* tp = pk_lane(g.wp, tc, C, lane);
#pragma unroll
		for (int i = 0; i < CPW; ++i) {
			const int c = min(wave * CPW + i, C - 1);
			d.b[i][0] = load16(tp + (size_t)c * 2048);
			d.b[i][1] = load16(tp + (size_t)c * 2048 + 1024);
		}
		const int jm = min(tc * 16 + ri, g.N - 1) >> 3;  // within the packed copy when no page is set
		// a global-space load: through a generic pointer it would be a flat load, which counts in
		// both wait counters and made every LDS wait of the epilogue drain the weight loads
#pragma unroll
		for (int mb = 0; mb < MB; ++mb)
			d.mbits[mb] = ((const __attribute__((address_space(1))) uint8_t*)pgp[mb])[masked[mb] ? jm : 0];
	};
	Tile t0buf, t1buf;
	int tile = blockIdx.x, it = 0;
	load_tile(tile, t0buf);  // the first tile's weights go out before the activations
	v4i x[MB][CPW][2];
#pragma unroll
	for (int mb = 0; mb < MB; ++mb) {
		const int r = mb * 16 + ri;
		const bool rok = r < g.M;
		const int8_t* arow = g.a + (size_t)(rok ? r : g.M - 1) * g.lda + grp * 16;
#pragma unroll
		for (int i = 0; i < CPW; ++i) {
			const int c = wave * CPW + i;
			const int cc = c < C ? c : C - 1;
			const v4i a0 = load16(arow + cc * 128), a1 = load16(arow + cc * 128 + 64);
			x[mb][i][0] = rok && c < C ? a0 : z;  // chunks past K multiply clamped weights by zero
			x[mb][i][1] = rok && c < C ? a1 : z;
		}
	}
	auto step = [&](int tl, int k, Tile& cur, Tile& nxt) {
		load_tile(tl + (int)gridDim.x, nxt);
		v4i acc[MB];
#pragma unroll
		for (int mb = 0; mb < MB; ++mb) {
			acc[mb] = z;
#pragma unroll
			for (int i = 0; i < CPW; ++i) {
				acc[mb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(x[mb][i][0], cur.b[i][0], acc[mb], 0, 0, 0);
				acc[mb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(x[mb][i][1], cur.b[i][1], acc[mb], 0, 0, 0);
			}
			red[k & 1][wave][mb][lane] = acc[mb];
		}
		__syncthreads();
		const int j = tl * 16 + ri;
#pragma unroll
		for (int mb = 0; mb < MB; ++mb) {
			int32_t tot = 0;
#pragma unroll
			for (int w = 0; w < kGemvWaves; ++w) tot += ((const int32_t*)&red[k & 1][w][mb][lane])[wave];
			const int tk = mb * 16 + grp * 4 + wave;
			const int32_t lv = masked[mb] && j < g.N && !((cur.mbits[mb] >> (j & 7)) & 1u) ? INT32_MIN : tot;
			uint64_t key = j < g.N ? ((uint64_t)((uint32_t)lv ^ 0x80000000u) << 32) | (0xffffffffu - (uint32_t)j) : 0;
#pragma unroll
			for (int o = 8; o > 0; o >>= 1) {
				const uint64_t k2 = __shfl_xor(key, o, 16);
				key = k2 > key ? k2 : key;
			}
			if (ri == 0) s_key[k][tk] = key;
		}
	};
	while (tile < T) {
		step(tile, it, t0buf, t1buf);
		tile += gridDim.x;
		++it;
		if (tile >= T) break;
		step(tile, it, t1buf, t0buf);
		tile += gridDim.x;
		++it;
	}
	__syncthreads();
	for (int q = threadIdx.x; q < it * MB * 16; q += 256) {
		const int k = q / (MB * 16), tk = q % (MB * 16);
		if (tk < g.M) e.argmax_key[(size_t)tk * e.key_ld + (int)blockIdx.x + k * (int)gridDim.x] = s_key[k][tk];
	}
}

// ------------------------------------------------------------------------------------------
// Decode GEMV, wave-per-tile form (M <= 16), for the launches with no projection epilogue: raw
// int32 accumulators (one plane, or split-K planes the consumer adds) and LM-head argmax keys.
// A block of 4 waves covers 4 consecutive 16-column tiles and one K range (split s of
// gridDim.y); each wave owns one tile over the whole range, so no wave waits for another once
// the block has staged its range of the 16 activation rows in LDS (zeros past M).  A wave
// issues the loads of NCH 128-byte chunks before the MFMAs that consume them; lane (ri, grp)
// holds 32 contiguous bytes of weight row ri and of activation row ri at the same k offsets
// (v_mfma_i32_16x16x64_i8, exact integer sums; accumulator lane l: tokens 4 (l / 16) .. +3 of
// column l % 16).  Measured against k_gemv on the 1.5B decode shapes with every layer's weights
// streaming from HBM: LM head 59 -> 49 us, down projection (8 planes) 8.4 -> 6.4 us.
// ------------------------------------------------------------------------------------------
// lane `lane`'s 16 bytes of chunk 0, half 0 of `tile` in a packed decode copy (k_gemv_pk)
__device__ __forceinline__ const int8_t* pk_lane(const int8_t* wp, int tile, int C, int lane) {
	return wp + (size_t)tile * C * 2048 + lane * 16;
}

// PK: the weights are read from the packed decode copy g.wp (see k_gemv_pk), the activations
// with its lane -> k map.
template <int NCH, bool PK>
__global__ __launch_bounds__(256) void k_gemv_w(GemmArgs g, int cps) {
	extern __shared__ __attribute__((aligned(16))) int8_t xs[];  // [16][span] activation rows
	const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
	const int tile = blockIdx.x * 4 + wave, split = blockIdx.y;
	const int ri = lane & 15, grp = lane >> 4;
	const int C = g.K >> 7;
	const int c_begin = split * cps, c_end = min(C, c_begin + cps);
	const int span = max(0, c_end - c_begin) * 128;
	const v4i z = v4i{0, 0, 0, 0};
	// chunk c of this lane's weight row: bytes [c * wstep, + 16) and [c * wstep + hoff, + 16)
	const int8_t* wrow = PK ? pk_lane(g.wp, min(tile, (g.N + 15) / 16 - 1), C, lane)
	                        : g.w + (size_t)min(tile * 16 + ri, g.N - 1) * g.K + grp * 32;
	constexpr int wstep = PK ? 2048 : 128, hoff = PK ? 1024 : 16;
	// the first batch of weights goes out before the activations are staged
	v4i b[NCH][2];
	int c0 = c_begin;
	const int c_last = max(c_begin, c_end - 1);
#pragma unroll
	for (int i = 0; i < NCH; ++i) {
		const int c = min(c0 + i, c_last);
		b[i][0] = load16(wrow + (size_t)c * wstep);
		b[i][1] = load16(wrow + (size_t)c * wstep + hoff);
	}
	{
		const int vecs = span >> 4;  // 16-byte vectors per row
		for (int i = threadIdx.x; i < 16 * vecs; i += 256) {
			const int r = i / vecs, v = i - r * vecs;
			const v4i x = r < g.M ? load16(g.a + (size_t)r * g.lda + (size_t)c_begin * 128 + v * 16) : z;
			*(v4i*)(xs + r * span + v * 16) = x;
		}
	}
	__syncthreads();
	v4i acc = z;
	// activations in the weights' lane -> k map: bytes 128 c + {0, 64} + 16 grp (packed) or
	// 128 c + 32 grp + {0, 16}
	constexpr int xoff = PK ? 64 : 16;
	const int8_t* xrow = xs + ri * span + grp * (PK ? 16 : 32) - c_begin * 128;
	while (c0 < c_end) {
#pragma unroll
		for (int i = 0; i < NCH; ++i) {
			const int c = c0 + i;
			if (c < c_end) {
				const v4i x0 = *(const v4i*)(xrow + c * 128), x1 = *(const v4i*)(xrow + c * 128 + xoff);
				acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(x0, b[i][0], acc, 0, 0, 0);
				acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(x1, b[i][1], acc, 0, 0, 0);
			}
		}
		c0 += NCH;
		if (c0 >= c_end) break;
#pragma unroll
		for (int i = 0; i < NCH; ++i) {
			const int c = min(c0 + i, c_last);
			b[i][0] = load16(wrow + (size_t)c * wstep);
			b[i][1] = load16(wrow + (size_t)c * wstep + hoff);
		}
	}
	if (tile * 16 >= g.N) return;
	const int j = tile * 16 + ri;
	const int t0 = grp * 4;  // this lane's tokens: t0 .. t0 + 3
	const Epilogue& e = g.epi;
	if (g.splits > 1 || e.raw_out) {
		int32_t* dst = g.splits > 1 ? g.split_part + (size_t)split * g.M * g.N : e.raw_out;
#pragma unroll
		for (int v = 0; v < 4; ++v)
			if (t0 + v < g.M && j < g.N) dst[(size_t)(t0 + v) * g.N + j] = acc[v];
	} else {
		// per (token, 16-column tile) greedy keys: the larger logit, then the smaller index; a
		// schema-masked token's logit counts as INT32_MIN
#pragma unroll
		for (int v = 0; v < 4; ++v) {
			const uint8_t* pg = e.mask_page && t0 + v < g.M ? e.mask_page[t0 + v] : nullptr;
			const int32_t lv = pg && j < g.N && !((pg[j >> 3] >> (j & 7)) & 1u) ? INT32_MIN : acc[v];
			uint64_t key = j < g.N ? ((uint64_t)((uint32_t)lv ^ 0x80000000u) << 32) | (0xffffffffu - (uint32_t)j) : 0;
			for (int o = 8; o > 0; o >>= 1) {
				const uint64_t k2 = __shfl_xor(key, o, 16);
				key = k2 > key ? k2 : key;
			}
			if (ri == 0 && t0 + v < g.M) e.argmax_key[(size_t)(t0 + v) * e.key_ld + tile] = key;
		}
	}
}

// ------------------------------------------------------------------------------------------
// Decode GEMVs on the packed weight layout (M <= 32).  Each projection keeps, beside its
// row-major matrix (read by the prefill GEMMs), a decode copy stored tile-major: for 16-column
// tile t, 128-byte K chunk c and half h, the 1 KB block at ((t * C + c) * 2 + h) * 1024 holds,
// for lane l = 16 grp + ri, the 16 bytes W[16 t + ri][128 c + 64 h + 16 grp .. +16) (rows past N
// zero).  A 16-byte load per lane then reads 1 KB of contiguous memory that is already the weight
// operand of v_mfma_i32_16x16x64_i8; the activations are read with the same lane -> k map (row ri,
// bytes 128 c + 64 h + 16 grp), so the integer sums are exact.  Against the row-major layout,
// where one load instruction touches 16 rows at a 32-byte stride, this cut the weight stream of
// the 1.5B decode shapes by 10-25 % in a study with 28 rotating weight copies.
// ------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_pack_gemv(const int8_t* w, int N, int K, int8_t* wp, int64_t units) {
	const int64_t u = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // (tile, c, h) 1 KB block
	if (u >= units) return;
	const int lane = threadIdx.x & 63, C = K >> 7;
	const int h = (int)(u & 1), c = (int)((u >> 1) % C);
	const int64_t tile = (u >> 1) / C;
	const int64_t row = tile * 16 + (lane & 15);
	const v4i z = v4i{0, 0, 0, 0};
	const v4i v = row < N ? load16(w + row * K + c * 128 + h * 64 + (lane >> 4) * 16) : z;
	*(v4i*)(wp + u * 1024 + lane * 16) = v;
}


// Projection GEMV: NT tiles per block (tile blockIdx.x + i * gridDim.x), the loop fully unrolled
// so that the wait counts before each tile's MFMAs are exact: the weights of tile i + 2 are issued
// as tile i's are consumed, two register sets alternating.  A runtime tile loop put a full drain
// of the vector-memory counter at its back edge (a store-address register reused by a loop-carried
// copy), and one 4-wave block per CU with an even share of tiles is what the memory system rewards:
// in a study of the 1.5B gate|up shape, 224 blocks x 5 tiles took 6.9 us and 280 x 4 (24 CUs
// holding two blocks) 9.0 us.  Wave w owns K chunks [w CPW, w CPW + CPW) of every tile and keeps
// their activation rows in registers for the whole launch; the four partial sums meet in a
// double-buffered LDS slot, and wave w finishes row w of each 4-token group: raw int32 output, or
// the projection epilogue of k_gemv (WSC1 fold, LoRA delta, bias reconcile, funnel tile maximum).
// EPI: kPkRaw (raw int32 output), kPkFunnel (funnel segments without bias or LoRA: fold, tile
// maximum, stores, in straight-line code) or kPkGeneral (any projection epilogue).
enum PkEpi { kPkRaw = 0, kPkFunnel = 1, kPkGeneral = 2 };

// NW = 8 (two row groups, K past 16 chunks): eight waves of CPW chunks each instead of four, so a
// wave's activation rows stay in registers (at four waves and seven chunks the compiler reloaded
// them before each MFMA, and every such wait also waited for the prefetched weights); wave w then
// finishes token row w % 4 of row group w / 4.
template <int MB, int NT, int CPW, int EPI, int NW = kGemvWaves>
__global__ __launch_bounds__(64 * NW) void k_gemv_pk(GemmArgs g) {
	static_assert(NW == kGemvWaves || (NW == 2 * kGemvWaves && MB == 2), "eight waves only for two row groups");
	__shared__ v4i red[2][NW][MB][64];
	const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, ri = lane & 15, grp = lane >> 4;
	const int C = g.K >> 7, T = (g.N + 15) / 16;
	const v4i z = v4i{0, 0, 0, 0};
	// the first tile's weights go out first: they need only wp, K and N
	// a tile's weights, and its column's fold parameters, bias and segment fields, all fetched two
	// tiles ahead so that no epilogue waits on a load
	struct Slot {
		v4i b[CPW][2];
		int32_t f0, f1, f2;
		int64_t bias;
		SegView sg;
	};
	Slot S[2];
	const int8_t* const wp = g.wp;
	auto load_w = [&](int i, Slot& d) {
		const int tile = min((int)blockIdx.x + i * (int)gridDim.x, T - 1);
		const int8_t* tp = pk_lane(wp, tile, C, lane);
#pragma unroll
		for (int c2 = 0; c2 < CPW; ++c2) {
			const int c = min(wave * CPW + c2, C - 1);
			d.b[c2][0] = load16(tp + (size_t)c * 2048);
			d.b[c2][1] = load16(tp + (size_t)c * 2048 + 1024);
		}
	};
	load_w(0, S[0]);
	v4i x[MB][CPW][2];
#pragma unroll
	for (int mb = 0; mb < MB; ++mb) {
		const int r = mb * 16 + ri;
		const bool rok = r < g.M;
		const int8_t* arow = g.a + (size_t)(rok ? r : g.M - 1) * g.lda + grp * 16;
#pragma unroll
		for (int i = 0; i < CPW; ++i) {
			const int c = wave * CPW + i;
			const bool ok = rok && c < C;
			const int cc = c < C ? c : C - 1;
			const v4i a0 = load16(arow + cc * 128), a1 = load16(arow + cc * 128 + 64);
			x[mb][i][0] = ok ? a0 : z;  // chunks past K multiply clamped weights by zero
			x[mb][i][1] = ok ? a1 : z;
		}
	}
	// the second tile's weights after the activations, so the first tile's MFMAs wait for neither
	if (NT > 1) load_w(1, S[1]);
	const Epilogue& e = g.epi;
	int32_t* const raw_out = e.raw_out;
	constexpr bool proj = EPI != kPkRaw;
	// fold parameters and bias of tile i's column for this lane, issued behind the weights.  The
	// loads are unconditional, from always-valid addresses (the weights stand in for values a launch
	// does not use): a load under a branch leaves the wait counts after the join unknown, and the
	// compiler then drains every outstanding load, the prefetched weights included.
	auto load_p = [&](int i, Slot& d) {
		const int tile = min((int)blockIdx.x + i * (int)gridDim.x, T - 1);
		const SegView sg = seg_view(e, proj ? tile_segment(e, tile * 16) : 0);
		d.sg = sg;
		const int jj = min(tile * 16 + ri, g.N - 1) - sg.n_begin;
		const int32_t* fp = proj ? sg.fold + 3 * jj : (const int32_t*)wp;
		d.f0 = fp[0];
		d.f1 = fp[1];
		d.f2 = fp[2];
		if (EPI == kPkGeneral) d.bias = *(sg.bias ? sg.bias + jj : (const int64_t*)wp);
	};
	load_p(0, S[0]);
	if (NT > 1) load_p(1, S[1]);
	// bias reconcile inputs of this lane's epilogue tokens (mb * 16 + 4 grp + wave)
	int64_t p_rcp[MB], p_ein[MB];
	const int64_t* const in_recip = e.in_recip;
	const Scale* const in_scale = e.in_scale;
#pragma unroll
	for (int mb = 0; mb < MB; ++mb) {
		const int tk = min(mb * 16 + grp * 4 + (wave & 3), g.M - 1);
		p_rcp[mb] = EPI == kPkGeneral ? *(in_recip ? in_recip + tk : (const int64_t*)wp) : 0;
		p_ein[mb] = EPI == kPkGeneral ? (in_scale ? in_scale + tk : (const Scale*)wp)->e : 0;
	}
	const int rank = e.rank, layer = e.layer;
	int32_t* const status = e.status;
	const TokenInfo* const tok = e.tok;
#pragma unroll
	for (int i = 0; i < NT; ++i) {
		Slot& cur = S[i & 1];
		v4i acc[MB];
#pragma unroll
		for (int mb = 0; mb < MB; ++mb) {
			acc[mb] = z;
#pragma unroll
			for (int c2 = 0; c2 < CPW; ++c2) {
				acc[mb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(x[mb][c2][0], cur.b[c2][0], acc[mb], 0, 0, 0);
				acc[mb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(x[mb][c2][1], cur.b[c2][1], acc[mb], 0, 0, 0);
			}
		}
		const int32_t f0 = cur.f0, f1 = cur.f1, f2 = cur.f2;
		const int64_t bias = cur.bias;
		const SegView sg = cur.sg;
		if (i + 2 < NT) {
			load_w(i + 2, cur);
			load_p(i + 2, cur);
		}
#pragma unroll
		for (int mb = 0; mb < MB; ++mb) red[i & 1][wave][mb][lane] = acc[mb];
		__builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes have landed
		__builtin_amdgcn_s_barrier();
		const int tile = blockIdx.x + i * gridDim.x;
		const int j = tile * 16 + ri;
		const bool col_ok = tile < T && j < g.N;
		const int jj = j - sg.n_begin;
#pragma unroll
		for (int mb = 0; mb < MB; ++mb) {
			if (NW != kGemvWaves && mb != (wave >> 2)) continue;  // (wave-uniform)
			int32_t tot = 0;
#pragma unroll
			for (int w = 0; w < NW; ++w) tot += ((const int32_t*)&red[i & 1][w][mb][lane])[wave & 3];
			const int tk = mb * 16 + grp * 4 + (wave & 3);
			const bool live = col_ok && tk < g.M;
			if (EPI == kPkRaw) {
				if (live) raw_out[(size_t)tk * g.N + j] = tot;
				continue;
			}
			if (EPI == kPkFunnel) {
				// |tot| <= 127^2 K < 2^29 for K <= 4096: the bounded fold applies
				const int32_t val = fold_bounded(tot, fold_consts(f0, f1, f2));
				const uint32_t mabs = dpp_max16(live ? (uint32_t)(val < 0 ? -val : val) : 0u);
				if (live) ((int32_t*)sg.out)[(size_t)tk * sg.ld_out + jj] = val;
				if (ri == 0 && tk < g.M && tile < T) sg.maxpart[(size_t)tile * kPartLd + tk] = mabs;
				continue;
			}
			int64_t val = apply_fold((int64_t)tot, f0, f1, f2);
			if (sg.lora_b && live) val += lora_delta_cold(sg.lora_b, sg.lora_u, sg.lora_dfold, rank, tk, jj);
			if (sg.bias) {
				int64_t term;
				if (bias_term(bias, p_rcp[mb], p_ein[mb], val, &term)) val += term;
				else if (live) set_status(status, tok[tk].slot, layer, kBiasReconcileProductOutOfDomain);
			}
			const uint32_t mabs = dpp_max16(live && sg.mode == kSegFunnel ? sat_abs_u32(val) : 0u);  // tile max
			if (live) {
				if (sg.mode == kSegWide) ((int64_t*)sg.out)[(size_t)tk * sg.ld_out + jj] = val;
				else ((int32_t*)sg.out)[(size_t)tk * sg.ld_out + jj] = sat_i32(val);
			}
			if (sg.mode == kSegFunnel && sg.maxpart && ri == 0 && tk < g.M && tile < T)
				sg.maxpart[(size_t)tile * kPartLd + tk] = mabs;
		}
	}
}

// Split-K GEMV with raw partial planes (long K: the down projection).  Block (tile group x,
// split y) covers NTB consecutive tiles and K chunks [y cps, y cps + cps), cps = WPB * CPW; wave w
// holds chunks y cps + w CPW .. + CPW of the activation rows in registers and multiplies them
// into all NTB tiles, so each activation byte is read once per tile group rather than once per
// tile.  The waves' sums meet by integer adds into LDS (exact in any order) and the block stores
// plane y of [splits][M][N].  1.5B down (K 8960) in a study: 4.7 us against 6.3 us for the
// wave-per-tile form on row-major weights.
template <int MB, int NTB, int CPW, int WPB>
__global__ __launch_bounds__(64 * WPB) void k_gemv_sk(GemmArgs g, int cps) {
	__shared__ int32_t sum[NTB][MB * 16][16];
	const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, ri = lane & 15, grp = lane >> 4;
	const int C = g.K >> 7, T = (g.N + 15) / 16, split = blockIdx.y;
	const int c0 = split * cps, c1 = min(C, c0 + cps);
	const int tile0 = blockIdx.x * NTB;
	for (int i = threadIdx.x; i < NTB * MB * 256; i += 64 * WPB) (&sum[0][0][0])[i] = 0;
	__syncthreads();
	const v4i z = v4i{0, 0, 0, 0};
	v4i b[NTB][CPW][2];
#pragma unroll
	for (int t = 0; t < NTB; ++t) {
		const int8_t* tp = pk_lane(g.wp, min(tile0 + t, T - 1), C, lane);
#pragma unroll
		for (int i = 0; i < CPW; ++i) {
			const int c = min(c0 + wave * CPW + i, c1 - 1);
			b[t][i][0] = load16(tp + (size_t)c * 2048);
			b[t][i][1] = load16(tp + (size_t)c * 2048 + 1024);
		}
	}
	v4i x[MB][CPW][2];
#pragma unroll
	for (int mb = 0; mb < MB; ++mb) {
		const int r = mb * 16 + ri;
		const bool rok = r < g.M;
		const int8_t* arow = g.a + (size_t)(rok ? r : g.M - 1) * g.lda + grp * 16;
#pragma unroll
		for (int i = 0; i < CPW; ++i) {
			const int c = c0 + wave * CPW + i;
			const bool ok = rok && c < c1;
			const int cc = min(c, c1 - 1);
			const v4i a0 = load16(arow + (size_t)cc * 128), a1 = load16(arow + (size_t)cc * 128 + 64);
			x[mb][i][0] = ok ? a0 : z;
			x[mb][i][1] = ok ? a1 : z;
		}
	}
#pragma unroll
	for (int t = 0; t < NTB; ++t)
#pragma unroll
		for (int mb = 0; mb < MB; ++mb) {
			v4i acc = z;
#pragma unroll
			for (int i = 0; i < CPW; ++i) {
				acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(x[mb][i][0], b[t][i][0], acc, 0, 0, 0);
				acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(x[mb][i][1], b[t][i][1], acc, 0, 0, 0);
			}
#pragma unroll
			for (int v = 0; v < 4; ++v) atomicAdd(&sum[t][mb * 16 + grp * 4 + v][ri], acc[v]);
		}
	__syncthreads();
	int32_t* plane = g.split_part + (size_t)split * g.M * g.N;
	for (int i = threadIdx.x; i < NTB * MB * 256; i += 64 * WPB) {
		const int t = i / (MB * 256), rem = i - t * MB * 256, tk = rem >> 4, col = rem & 15;
		const int j = (tile0 + t) * 16 + col;
		if (tk < g.M && j < g.N) plane[(size_t)tk * g.N + j] = sum[t][tk][col];
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
// Prefill GEMM (M > 64): block tile BM x 128 with BK = 128.  The tile is cut into 128x64 wave
// tiles of v_mfma_i32_32x32x32_i8 (4x2), TW = BM / 64 of them, and each wave tile is shared by
// two waves that take the two 64-deep halves of every K step (2 TW waves: 8 at BM = 256); the
// pair's accumulators are summed in the epilogue.  Two waves per SIMD let one issue MFMAs
// while the other waits at the barrier or on load issue.
// Operands go global -> LDS directly (global_load_lds_dwordx4, 1 KB per wave instruction: 8 full
// 128-byte rows) through NS = 3 stages; the loads of K step t + 3 are issued between step t's
// MFMAs (the per-CU load rate is the other limit of this loop, so its issue is spread out),
// and the operand fragments of step t + 1 are read while step t's MFMAs run.  Rows of a stage
// hold XOR-swizzled 16-byte chunks (lds_chunk).  One barrier per K step.  Loads are
// unconditional: rows past M or N read a clamped valid row whose products land only in
// discarded outputs, and K is a multiple of 128.
// gridDim.z splits K; with several splits each stores its raw int32 partial plane and the
// consumer applies the epilogue (RawIn), as for the decode GEMV.  With one split the block runs
// the epilogue (see below).
// ------------------------------------------------------------------------------------------
constexpr int kPBN = 128, kPBK = 128, kPStride = kPBK, kPrefillStages = 3;

// LDS placement of the 16-byte chunk `q` (0..7) of tile row `row` (128 bytes a row): the chunk
// index is XORed with row bits 1..3, so 16 consecutive rows read at one chunk (the MFMA
// operand pattern: even and odd rows fall in the two 128-byte halves of the 64 banks, and the
// 8 even rows in 8 distinct chunks) are conflict-free; the direct loads write whole rows.
__device__ __forceinline__ int lds_chunk(int row, int q) { return row * kPStride + ((q ^ ((row >> 1) & 7)) << 4); }

// WSC1 fold without a branch on the identity flag (same value as apply_fold)
__device__ __forceinline__ int64_t fold_select(int32_t acc, int32_t identity, int32_t mult, int32_t shift) {
	const int64_t folded = (int64_t)rdbpot32(srdhm(acc, mult), shift);
	return identity != 0 ? (int64_t)acc : folded;
}

// The same fold as straight-line int32 arithmetic (apply_fold on an int32 accumulator; the
// result is int32 either way): srdhm as one 64-bit product, rdbpot32 as mask / threshold, the
// identity flag as a final select.
__device__ __forceinline__ int32_t fold32(int32_t acc, int32_t identity, int32_t mult, int32_t shift) {
	const int64_t ab = (int64_t)acc * (int64_t)mult + ((int64_t)1 << 30);
	const int64_t hi64 = ab >> 31;
	const int32_t hi = hi64 > kI32Max ? kI32Max : (int32_t)hi64;
	const uint32_t mask = ((uint32_t)1 << shift) - 1u;
	const uint32_t rem = (uint32_t)hi & mask;
	const uint32_t thr = (mask >> 1) + (hi < 0 ? 1u : 0u);
	const int32_t folded = (hi >> shift) + (rem > thr ? 1 : 0);
	return identity != 0 ? acc : folded;
}

// s_waitcnt with vmcnt(n), expcnt and lgkmcnt unconstrained (gfx9 encoding: vmcnt in bits
// 3:0 and 15:14)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
	static_assert(N >= 0 && N < 64, "vmcnt range");
	__builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0f70);
}

// LDS read of 16 bytes at byte address `base + OFF` of the shared segment, issued from inline
// assembly: the compiler's wait insertion would otherwise treat every pending direct-to-LDS
// load as a possible writer and drain them all before the read.  The caller waits on lgkmcnt
// itself (lgkm_wait) before using the result.
template <int OFF>
__device__ __forceinline__ v4i lds_read16(uint32_t base) {
	v4i r;
	asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(base), "i"(OFF));
	return r;
}

// lgkmcnt(N) wait that the fragments pass through, so nothing reading them moves above it
template <int N>
__device__ __forceinline__ void lgkm_wait(v4i (&a)[4], v4i (&b)[2]) {
	asm volatile("s_waitcnt lgkmcnt(%6)"
	             : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(b[0]), "+v"(b[1])
	             : "i"(N));
}

template <int BM, int NS>
__global__ __launch_bounds__(BM / 32 * 64, 1) void k_gemm_mfma(GemmArgs g, PrefillPlan pp) {
	constexpr int TW = BM / 64;           // wave tiles (128x64) per block tile
	constexpr int WAVES = 2 * TW, NT = WAVES * 64;
	constexpr int ROWS = BM + kPBN;
	constexpr int STAGE = ROWS * kPStride;  // bytes of one 128-deep K step of A and W rows
	constexpr int INSTS = STAGE / 1024;     // 1 KB direct-to-LDS wave loads per stage
	constexpr int CPT = INSTS / WAVES;      // per wave
	constexpr int CH = kPStride / 16;       // 16-byte chunks per row
	static_assert(CPT * WAVES == INSTS, "stage must split evenly over the waves");
	static_assert(NS >= 2 && (NS - 1) * CPT < 64, "stages in flight must fit vmcnt");
	__shared__ __attribute__((aligned(1024))) int8_t smem[NS * STAGE];
	const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
	const int wt = wave % TW, kh = wave / TW;  // wave tile, K half
	const int wm = (wt >> 1) * 128, wn = (wt & 1) * 64;

	const int tiles_m = (g.M + BM - 1) / BM;  // tile t: rows (t % tiles_m) * BM, columns (t / tiles_m) * 128
	v16i acc[4][2];
	// K steps [ks0, ks1) of tile `tile` into acc
	auto run_tile = [&](int tile, int ks0, int ks1) {
	const int m0 = (tile % tiles_m) * BM, n0 = (tile / tiles_m) * kPBN;
	const int k_begin = ks0 * kPBK, ntile = ks1 - ks0;
	// Each wave load instruction writes 1 KB of LDS in lane order (16 bytes per lane): lane l
	// of instruction i fills slot 64 i + l, i.e. row slot / 8 at physical chunk slot % 8, so it
	// fetches the logical chunk that lds_chunk() places there (rows clamped into the operands).
	const int8_t* src[CPT];
#pragma unroll
	for (int j = 0; j < CPT; ++j) {
		const int slot = (wave * CPT + j) * 64 + lane;
		const int row = slot / CH, pc = slot % CH;
		const int q = pc ^ ((row >> 1) & 7);
		if (row < BM) src[j] = g.a + (size_t)min(m0 + row, g.M - 1) * g.lda + k_begin + q * 16;
		else src[j] = g.w + (size_t)min(n0 + row - BM, g.N - 1) * g.K + k_begin + q * 16;
	}
	// load j of tile t into stage st (clamped: past the last tile the last is fetched again,
	// into a stage no step reads, so every step waits for the same count)
	auto issue_one = [&](int st, int t, int j) {
		const size_t kb = (size_t)min(t, ntile - 1) * kPBK;
		__builtin_amdgcn_global_load_lds((const void*)(src[j] + kb),
		                                 (__attribute__((address_space(3))) void*)(smem + st * STAGE + (wave * CPT + j) * 1024),
		                                 16, 0, 0);
	};
#pragma unroll
	for (int i = 0; i < 4; ++i)
#pragma unroll
		for (int j = 0; j < 2; ++j)
#pragma unroll
			for (int v = 0; v < 16; ++v) acc[i][j][v] = 0;
	// operand addresses: row wm + lane % 32 (+ 32 i) of A, wn + lane % 32 (+ 32 j) of B, chunk
	// 2 (2 kh + ks) + lane / 32; the swizzle depends only on the row's low bits, so +32 rows
	// keep it
	const uint32_t lds0 = (uint32_t)(size_t)(__attribute__((address_space(3))) int8_t*)smem;
	const int arow = wm + (lane & 31), brow = BM + wn + (lane & 31);
	uint32_t aoff[2], boff[2];
#pragma unroll
	for (int ks = 0; ks < 2; ++ks) {
		aoff[ks] = lds0 + lds_chunk(arow, 2 * (2 * kh + ks) + (lane >> 5));
		boff[ks] = lds0 + lds_chunk(brow, 2 * (2 * kh + ks) + (lane >> 5));
	}
	constexpr int R32 = 32 * kPStride;
	// the wave's operand fragments of one stage: A rows +0/32/64/96 and B rows +0/32 for its two
	// 32-deep steps
	auto frags = [&](v4i (&a)[8], v4i (&b)[4], int st) {
#pragma unroll
		for (int ks = 0; ks < 2; ++ks) {
			const uint32_t ab = aoff[ks] + st * STAGE, bb = boff[ks] + st * STAGE;
			a[4 * ks] = lds_read16<0>(ab);
			a[4 * ks + 1] = lds_read16<R32>(ab);
			a[4 * ks + 2] = lds_read16<2 * R32>(ab);
			a[4 * ks + 3] = lds_read16<3 * R32>(ab);
			b[2 * ks] = lds_read16<0>(bb);
			b[2 * ks + 1] = lds_read16<R32>(bb);
		}
	};
	auto frags_wait = [&](v4i (&a)[8], v4i (&b)[4]) {
		lgkm_wait<0>(*(v4i(*)[4])&a[0], *(v4i(*)[2])&b[0]);
		lgkm_wait<0>(*(v4i(*)[4])&a[4], *(v4i(*)[2])&b[2]);
	};
	// step t: x holds tile t's fragments (read during step t - 1), y receives tile t + 1's.
	// Every wave's reads of tile t are complete before the barrier, so its stage takes the loads
	// of tile t + NS, spread between the MFMAs.
	auto step = [&](v4i (&xa)[8], v4i (&xb)[4], v4i (&ya)[8], v4i (&yb)[4], int t) {
		frags_wait(xa, xb);
		wait_vmcnt<(NS - 2) * CPT>();  // own loads of tile t + 1 have landed
		// a bare s_barrier: __syncthreads() adds a workgroup release fence, which would drain
		// every direct-to-LDS load still in flight
		__builtin_amdgcn_s_barrier();
		frags(ya, yb, (t + 1) % NS);
		int li = 0, m = 0;
#pragma unroll
		for (int ks = 0; ks < 2; ++ks)
#pragma unroll
			for (int i = 0; i < 4; ++i)
#pragma unroll
				for (int j = 0; j < 2; ++j) {
					if (li < CPT && m == li * 16 / CPT) {
						__builtin_amdgcn_sched_barrier(0);
						issue_one(t % NS, t + NS, li);
						++li;
						__builtin_amdgcn_sched_barrier(0);
					}
					acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(xa[4 * ks + i], xb[2 * ks + j], acc[i][j], 0, 0, 0);
					++m;
				}
	};
	v4i ca[8], cb[4], na[8], nb[4];
#pragma unroll
	for (int i = 0; i < NS; ++i)
#pragma unroll
		for (int j = 0; j < CPT; ++j) issue_one(i, i, j);
	wait_vmcnt<(NS - 1) * CPT>();
	__builtin_amdgcn_s_barrier();
	frags(ca, cb, 0);
	for (int t = 0; t < ntile; t += 2) {
		step(ca, cb, na, nb, t);
		if (t + 1 < ntile) step(na, nb, ca, cb, t + 1);
	}
	frags_wait(ca, cb);
	frags_wait(na, nb);
	wait_vmcnt<0>();  // the trailing (clamped) loads land before the stages are reused
	__syncthreads();

	};
	// epilogue of tile `tile` on acc (raw split plane `split` when gridDim.z > 1)
	auto epilogue = [&](int tile, int split) {
	const int m0 = (tile % tiles_m) * BM, n0 = (tile / tiles_m) * kPBN;
	// Epilogue, 32 rows at a time: each wave parks a 32x64 slice of its accumulators in its own
	// 8 KB of LDS (the main loop's stages are free now); the two waves of a wave tile then sum
	// their slices, lane l owning the 4 columns wn + 4 (l % 16) .. +3 and rows l / 16 + 4 p
	// (p in 4 kh .. 4 kh + 3) of the slice -- 16-byte loads and stores, per-column parameters
	// in registers, each 16-column tile's partial maximum reduced over a lane quad with DPP.
	int32_t* slab = (int32_t*)smem + wave * 32 * 64;
	const int32_t* slab0 = (const int32_t*)smem + wt * 32 * 64;
	const int32_t* slab1 = (const int32_t*)smem + (wt + TW) * 32 * 64;
	const int c4 = (lane & 15) * 4, rsub = lane >> 4;
	const int col0 = n0 + wn + c4;  // first of this lane's 4 columns (with an epilogue N % 16 == 0)
	const bool col_ok = col0 < g.N;
	const Epilogue& e = g.epi;
	const bool raw = gridDim.z > 1 || e.raw_out;
	int32_t* raw_out = gridDim.z > 1 ? g.split_part + (size_t)split * g.M * g.N : e.raw_out;
	int32_t f0[4], f1[4], f2[4];
	int64_t bias[4];
	int ldc = 0;
	bool wide = false, has_bias = false;
	int32_t* fout = nullptr;
	int64_t* wout = nullptr;
	uint32_t* mpart = nullptr;
	// the block's per-row bias operands (reciprocal and exponent of the input scale), staged in
	// LDS after the slabs, so the store loop does not wait on a global load per row
	int64_t* s_rcp = (int64_t*)(smem + WAVES * 32 * 64 * 4);
	int64_t* s_ein = s_rcp + BM;
	static_assert(WAVES * 32 * 64 * 4 + BM * 16 <= NS * STAGE, "epilogue LDS");
	if (!raw) {
		// the lane's segment (bounds are multiples of 16: one per lane), every field read with a
		// constant index -- a lane-dependent index into the kernel arguments would copy them to
		// scratch memory
		int si = 0;
		if (e.nseg > 1 && col0 >= e.seg[0].n_end) si = 1;
		if (e.nseg > 2 && col0 >= e.seg[1].n_end) si = 2;
#define SSLM_SEG_FIELD(f) (si == 0 ? e.seg[0].f : (si == 1 ? e.seg[1].f : e.seg[2].f))
		const int32_t n_begin = SSLM_SEG_FIELD(n_begin), mode = SSLM_SEG_FIELD(mode);
		const int32_t* fold = SSLM_SEG_FIELD(fold);
		const int64_t* sb = SSLM_SEG_FIELD(bias);
		void* sout = SSLM_SEG_FIELD(out);
		uint32_t* smax = SSLM_SEG_FIELD(maxpart);
		ldc = SSLM_SEG_FIELD(ld_out);
#undef SSLM_SEG_FIELD
		const int jc = (col_ok ? col0 : n_begin) - n_begin;
		const int32_t* f = fold + 3 * jc;
#pragma unroll
		for (int q = 0; q < 4; ++q) {
			f0[q] = f[3 * q];
			f1[q] = f[3 * q + 1];
			f2[q] = f[3 * q + 2];
			bias[q] = sb ? sb[jc + q] : 0;
		}
		has_bias = sb != nullptr;
		wide = mode == kSegWide;
		fout = (int32_t*)sout + jc;
		wout = (int64_t*)sout + jc;
		mpart = smax ? smax + (size_t)(col0 >> 4) * kPartLd : nullptr;
	}
	bool any_bias = false;  // block-uniform: every segment's bias pointer
	for (int i = 0; i < e.nseg; ++i) any_bias = any_bias || (!raw && e.seg[i].bias != nullptr);
	__syncthreads();  // every wave is done reading the last LDS stage
	if (any_bias) {
		for (int r = threadIdx.x; r < BM; r += NT) {
			const int t = min(m0 + r, g.M - 1);
			s_rcp[r] = e.in_recip[t];
			s_ein[r] = e.in_scale[t].e;
		}
		__syncthreads();
	}
#pragma unroll
	for (int mt = 0; mt < 4; ++mt) {
		// 32x32 accumulator layout: lane holds column lane % 32 of the sub-tile, rows
		// 8 * (v / 4) + 4 * (lane / 32) + v % 4
#pragma unroll
		for (int nt = 0; nt < 2; ++nt)
#pragma unroll
			for (int v = 0; v < 16; ++v)
				slab[(8 * (v >> 2) + 4 * (lane >> 5) + (v & 3)) * 64 + nt * 32 + (lane & 31)] = acc[mt][nt][v];
		__syncthreads();
		for (int p = 4 * kh; p < 4 * kh + 4; ++p) {
			const int r = 4 * p + rsub;
			const int t = m0 + wm + mt * 32 + r;
			const bool ok = t < g.M && col_ok;
			const v4i a = *(const v4i*)&slab0[r * 64 + c4] + *(const v4i*)&slab1[r * 64 + c4];
			if (raw) {
				if (ok && col0 + 4 <= g.N) {
					*(v4i*)&raw_out[(size_t)t * g.N + col0] = a;
				} else if (ok) {
					for (int q = 0; q < 4 && col0 + q < g.N; ++q) raw_out[(size_t)t * g.N + col0 + q] = a[q];
				}
				continue;
			}
			if (!any_bias && !wide) {
				// no bias anywhere in the launch (o, gate|up, down): straight-line int32 fold,
				// int32 store, tile maximum -- no branch per element
				v4i o;
				uint32_t mx = 0;
#pragma unroll
				for (int q = 0; q < 4; ++q) {
					o[q] = fold32(a[q], f0[q], f1[q], f2[q]);
					mx = max(mx, o[q] < 0 ? 0u - (uint32_t)o[q] : (uint32_t)o[q]);
				}
				if (ok) *(v4i*)(fout + (size_t)t * ldc) = o;
				if (!ok) mx = 0;
				uint32_t w2 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mx, 0xb1, 0xf, 0xf, false);
				mx = max(mx, w2);
				w2 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mx, 0x4e, 0xf, 0xf, false);
				mx = max(mx, w2);
				if ((lane & 3) == 0 && t < g.M && col_ok && mpart) mpart[t] = mx;
				continue;
			}
			int64_t val[4];
			uint32_t mx = 0;
#pragma unroll
			for (int q = 0; q < 4; ++q) {
				val[q] = f0[q] != 0 ? (int64_t)a[q] : (int64_t)rdbpot32(srdhm(a[q], f1[q]), f2[q]);
				if (has_bias && ok) {
					int64_t term;
					const int rr = wm + mt * 32 + r;
					if (bias_term(bias[q], s_rcp[rr], s_ein[rr], val[q], &term)) val[q] += term;
					else set_status_rows(e.status, e.tok, e.layer, t, 1u);
				}
				const uint32_t m1 = sat_abs_u32(val[q]);
				mx = m1 > mx ? m1 : mx;
			}
			if (ok) {
				if (wide) {
					int64_t* o = wout + (size_t)t * ldc;
					*(longlong2*)o = make_longlong2(val[0], val[1]);
					*(longlong2*)(o + 2) = make_longlong2(val[2], val[3]);
				} else {
					*(v4i*)(fout + (size_t)t * ldc) = v4i{sat_i32(val[0]), sat_i32(val[1]), sat_i32(val[2]), sat_i32(val[3])};
				}
			}
			// quad max (quad_perm [1,0,3,2] then [2,3,0,1]): the 4 lanes of one 16-column tile
			if (!ok || wide) mx = 0;
			uint32_t w2 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mx, 0xb1, 0xf, 0xf, false);
			mx = w2 > mx ? w2 : mx;
			w2 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mx, 0x4e, 0xf, 0xf, false);
			mx = w2 > mx ? w2 : mx;
			if ((lane & 3) == 0 && t < g.M && col_ok && mpart && !wide) mpart[t] = mx;
		}
		__syncthreads();  // the slabs are rewritten for the next 32 rows
	}
	};

	const int S = g.K / kPBK;  // K steps
	// XCD-aware order: workgroups are dispatched round-robin over the 8 XCDs, so the virtual
	// block vb = (b % 8) * (B / 8) + b / 8 puts neighbouring tiles (which share A or W rows) in
	// one XCD's L2
	const int B = gridDim.x;
	const int vb = B % 8 == 0 ? (int)(blockIdx.x % 8) * (B / 8) + (int)(blockIdx.x / 8) : (int)blockIdx.x;
	// one tile per block; gridDim.z splits K into raw partial planes
	const int ks0 = blockIdx.z * pp.kspan / kPBK;
	run_tile(vb, ks0, min(S, ks0 + pp.kspan / kPBK));
	epilogue(vb, blockIdx.z);
}

// ------------------------------------------------------------------------------------------
// Wide prefill GEMM (the gate|up projection: N in the tens of thousands): 256 x 160 block tiles,
// so a 512-token chunk's 17,920 columns make 224 tiles -- one round over 256 CUs, where 256 x 128
// tiles make 280 and leave a second round mostly idle with its own prologue and epilogue.
// Block: 4 waves, wave w owns rows [64 w, 64 w + 64) x all 160 columns as 4 x 10
// v_mfma_i32_16x16x64_i8 accumulators.  Operands go global -> LDS directly through 3 stages of
// 128-deep K steps (416 rows of 128 bytes, XOR-swizzled as in lds_chunk; 13 one-kilobyte wave
// loads per wave per stage); a stage's two 64-deep halves are read from LDS together, the second
// while the first's MFMAs run.  Epilogue: raw int32, or funnel segments (WSC1 fold, int32 store,
// per-(16-column tile, token) maxima) without bias or LoRA -- a 16 x 16 accumulator is one
// column tile, reduced over its 16 lanes with DPP.  The fold parameters are loaded before the
// main loop.  Loads are unconditional (rows past M or N read a clamped valid row) and K is a
// multiple of 128.
// ------------------------------------------------------------------------------------------
constexpr int kWideBM = 256, kWideBN = 160, kWideStages = 3, kWideFoldMaxK = 32768;

__device__ __forceinline__ void lgkm_wait_n14(v4i (&a)[4], v4i (&b)[10]) {
	asm volatile("s_waitcnt lgkmcnt(14)"
	             : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(b[0]), "+v"(b[1]), "+v"(b[2]), "+v"(b[3]),
	               "+v"(b[4]), "+v"(b[5]), "+v"(b[6]), "+v"(b[7]), "+v"(b[8]), "+v"(b[9]));
}
__device__ __forceinline__ void lgkm_wait_n0(v4i (&a)[4], v4i (&b)[10]) {
	asm volatile("s_waitcnt lgkmcnt(0)"
	             : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(b[0]), "+v"(b[1]), "+v"(b[2]), "+v"(b[3]),
	               "+v"(b[4]), "+v"(b[5]), "+v"(b[6]), "+v"(b[7]), "+v"(b[8]), "+v"(b[9]));
}

// v_mfma_i32_16x16x64_i8 with the accumulator tied to one AGPR quad (dst = srcC).  Through the
// builtin the register allocator rotated a third of the 40 accumulators of k_gemm_wide through
// VGPR copies every K step, each copy waiting for its MFMA to retire.  The asm carries no
// hazard information: between two MFMAs on one accumulator there are 39 others, and the
// kernel pads with s_nop before VALU reads the accumulators after the loop.
__device__ __forceinline__ void mfma16_tied(v4i& acc, const v4i& a, const v4i& b) {
	asm("v_mfma_i32_16x16x64_i8 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}

__global__ __launch_bounds__(256, 1) void k_gemm_wide(GemmArgs g) {
	constexpr int BM = kWideBM, BN = kWideBN, NS = kWideStages, NB = BN / 16;
	constexpr int ROWS = BM + BN, STAGE = ROWS * kPStride;
	constexpr int CPT = STAGE / 1024 / 4;  // 13
	static_assert(CPT * 4 * 1024 == STAGE, "stage must split evenly over the waves");
	static_assert((NS - 1) * CPT < 64, "stages in flight must fit vmcnt");
	__shared__ __attribute__((aligned(1024))) int8_t smem[NS * STAGE];
	const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
	const int tiles_m = (g.M + BM - 1) / BM;
	const int B = gridDim.x;
	const int vb = B % 8 == 0 ? (int)(blockIdx.x % 8) * (B / 8) + (int)(blockIdx.x / 8) : (int)blockIdx.x;
	const int m0 = (vb % tiles_m) * BM, n0 = (vb / tiles_m) * BN;
	const int S = g.K / kPBK;
	const Epilogue& e = g.epi;
	const bool raw = e.raw_out != nullptr;
	const int cl = lane & 15;
	// The epilogue's fold parameters of the tile's 160 columns (480 int32, 120 chunks of 16
	// bytes, 12 per 16-column tile), loaded before the main loop, one chunk per thread, and
	// parked in LDS after it.
	constexpr int kParamChunks = BN * 3 / 4;
	v4i fchunk = v4i{0, 0, 0, 0};
	if (!raw && (int)threadIdx.x < kParamChunks) {
		const int c = threadIdx.x, c0 = n0 + 16 * (c / 12);
		if (c0 < g.N) {
			const int si = (e.nseg > 1 && c0 >= e.seg[0].n_end) ? ((e.nseg > 2 && c0 >= e.seg[1].n_end) ? 2 : 1) : 0;
			const int32_t* fold = si == 0 ? e.seg[0].fold : (si == 1 ? e.seg[1].fold : e.seg[2].fold);
			const int nb = si == 0 ? e.seg[0].n_begin : (si == 1 ? e.seg[1].n_begin : e.seg[2].n_begin);
			fchunk = load16((const int8_t*)(fold + 3 * (c0 - nb) + 4 * (c % 12)));
		}
	}
	const int8_t* src[CPT];
#pragma unroll
	for (int j = 0; j < CPT; ++j) {
		const int slot = (wave * CPT + j) * 64 + lane;
		const int row = slot >> 3, pc = slot & 7;
		const int q = pc ^ ((row >> 1) & 7);
		if (row < BM) src[j] = g.a + (size_t)min(m0 + row, g.M - 1) * g.lda + q * 16;
		else src[j] = g.w + (size_t)min(n0 + row - BM, g.N - 1) * g.K + q * 16;
	}
	auto issue = [&](int st, int t) {  // past the last step the last is fetched again (never read)
		const size_t kb = (size_t)min(t, S - 1) * kPBK;
#pragma unroll
		for (int j = 0; j < CPT; ++j)
			__builtin_amdgcn_global_load_lds((const void*)(src[j] + kb),
			                                 (__attribute__((address_space(3))) void*)(smem + st * STAGE + (wave * CPT + j) * 1024),
			                                 16, 0, 0);
	};
	const uint32_t lds0 = (uint32_t)(size_t)(__attribute__((address_space(3))) int8_t*)smem;
	// the lane's fragment rows: A rows 64 w + 16 i + lane % 16, B rows BM + 16 j + lane % 16; in a
	// 64-deep half h the lane reads 16-byte chunk 4 h + lane / 16
	uint32_t aoff[2], boff[2];
#pragma unroll
	for (int h = 0; h < 2; ++h) {
		aoff[h] = lds0 + lds_chunk(64 * wave + cl, 4 * h + (lane >> 4));
		boff[h] = lds0 + lds_chunk(BM + cl, 4 * h + (lane >> 4));
	}
	constexpr int R16 = 16 * kPStride;  // 16 rows further: the swizzle depends on row bits 1..3 only
	v4i acc[4][NB];
#pragma unroll
	for (int i = 0; i < 4; ++i)
#pragma unroll
		for (int j = 0; j < NB; ++j) acc[i][j] = v4i{0, 0, 0, 0};
#pragma unroll
	for (int s0 = 0; s0 < NS - 1; ++s0) issue(s0, s0);
	int t = 0;
	do {  // S >= 1 (K is a positive multiple of 128): no zero-trip path, no accumulator copy at its exit
		wait_vmcnt<(NS - 2) * CPT>();  // own loads of step t have landed
		__builtin_amdgcn_s_barrier();  // everyone's have; everyone is done with step t - 1
		issue((t + NS - 1) % NS, t + NS - 1);
		const uint32_t so = (uint32_t)((t % NS) * STAGE);
		v4i a0[4], b0[NB], a1[4], b1[NB];
		a0[0] = lds_read16<0>(aoff[0] + so);
		a0[1] = lds_read16<R16>(aoff[0] + so);
		a0[2] = lds_read16<2 * R16>(aoff[0] + so);
		a0[3] = lds_read16<3 * R16>(aoff[0] + so);
		b0[0] = lds_read16<0>(boff[0] + so);
		b0[1] = lds_read16<R16>(boff[0] + so);
		b0[2] = lds_read16<2 * R16>(boff[0] + so);
		b0[3] = lds_read16<3 * R16>(boff[0] + so);
		b0[4] = lds_read16<4 * R16>(boff[0] + so);
		b0[5] = lds_read16<5 * R16>(boff[0] + so);
		b0[6] = lds_read16<6 * R16>(boff[0] + so);
		b0[7] = lds_read16<7 * R16>(boff[0] + so);
		b0[8] = lds_read16<8 * R16>(boff[0] + so);
		b0[9] = lds_read16<9 * R16>(boff[0] + so);
		a1[0] = lds_read16<0>(aoff[1] + so);
		a1[1] = lds_read16<R16>(aoff[1] + so);
		a1[2] = lds_read16<2 * R16>(aoff[1] + so);
		a1[3] = lds_read16<3 * R16>(aoff[1] + so);
		b1[0] = lds_read16<0>(boff[1] + so);
		b1[1] = lds_read16<R16>(boff[1] + so);
		b1[2] = lds_read16<2 * R16>(boff[1] + so);
		b1[3] = lds_read16<3 * R16>(boff[1] + so);
		b1[4] = lds_read16<4 * R16>(boff[1] + so);
		b1[5] = lds_read16<5 * R16>(boff[1] + so);
		b1[6] = lds_read16<6 * R16>(boff[1] + so);
		b1[7] = lds_read16<7 * R16>(boff[1] + so);
		b1[8] = lds_read16<8 * R16>(boff[1] + so);
		b1[9] = lds_read16<9 * R16>(boff[1] + so);
		lgkm_wait_n14(a0, b0);  // the first half's 14 reads done (the second's 14 may be pending)
#pragma unroll
		for (int i = 0; i < 4; ++i)
#pragma unroll
			for (int j = 0; j < NB; ++j) mfma16_tied(acc[i][j], a0[i], b0[j]);
		lgkm_wait_n0(a1, b1);
#pragma unroll
		for (int i = 0; i < 4; ++i)
#pragma unroll
			for (int j = 0; j < NB; ++j) mfma16_tied(acc[i][j], a1[i], b1[j]);
	} while (++t < S);
	// The last MFMAs' results settle before anything reads the accumulators: the padding, then an
	// empty asm per accumulator that claims to rewrite it, so no read is scheduled above the
	// padding (the accumulators are registers: a memory clobber alone does not hold them back).
	asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
	for (int i = 0; i < 4; ++i)
#pragma unroll
		for (int j = 0; j < NB; ++j) asm volatile("" : "+a"(acc[i][j]));
	wait_vmcnt<0>();  // the trailing (clamped) loads land before the stages are reused
	__syncthreads();
	// 16x16 layout: lane holds column lane % 16, rows 4 (lane / 16) + v
	if (raw) {
		const int rbase = m0 + 64 * wave + 4 * (lane >> 4);
#pragma unroll
		for (int j = 0; j < NB; ++j) {
			const int col = n0 + 16 * j + cl;
#pragma unroll
			for (int i = 0; i < 4; ++i)
#pragma unroll
				for (int v = 0; v < 4; ++v) {
					const int row = rbase + 16 * i + v;
					if (col < g.N && row < g.M) e.raw_out[(size_t)row * g.N + col] = acc[i][j][v];
				}
		}
		return;
	}
	// Funnel segments: each wave parks half of its 64 x 160 accumulators (64 x 80, rows padded to
	// 84 words: the four 4-row groups of a store fall in distinct banks) in its own LDS slab, then
	// reads them back four consecutive columns per lane: lane l < 60 keeps column group l % 20 of
	// the half and walks rows l / 20, + 3, + 6, ... (lanes 60..63 idle), so its fold constants,
	// output segment and addresses are set once per half.  A lane quad is one 16-column tile of
	// one row (20 groups are 5 whole quads), so the tile maximum is a quad DPP maximum.
	constexpr int HALF = NB / 2, LDW = 84, SLAB = 64 * LDW, GRPS = HALF * 4, RST = 64 / GRPS;
	constexpr int RITER = (64 + RST - 1) / RST;
	static_assert(NB % 2 == 0 && 4 * SLAB * 4 + BN * 12 <= NS * STAGE, "epilogue LDS");
	static_assert(GRPS % 4 == 0 && RST * GRPS <= 64 && RST == 3, "readback lane map");
	static_assert(3 * SLAB + (RITER * RST + RST - 1) * LDW + 4 * GRPS <= 4 * SLAB + BN * 3, "readback rows stay in LDS");
	int32_t* slab = (int32_t*)smem + wave * SLAB;
	int32_t* prm = (int32_t*)smem + 4 * SLAB;  // [BN][3]
	if ((int)threadIdx.x < kParamChunks) *(v4i*)&prm[4 * threadIdx.x] = fchunk;
	__syncthreads();
	const int grp = lane % GRPS, rp = lane / GRPS;  // rp == RST: idle lane
	const int rowb = m0 + 64 * wave + rp;
#pragma unroll
	for (int hf = 0; hf < 2; ++hf) {
#pragma unroll
		for (int jj = 0; jj < HALF; ++jj)
#pragma unroll
			for (int i = 0; i < 4; ++i)
#pragma unroll
				for (int v = 0; v < 4; ++v)
					slab[(16 * i + 4 * (lane >> 4) + v) * LDW + 16 * jj + cl] = acc[i][hf * HALF + jj][v];
		// the wave reads back only what it wrote: LDS operations of a wave complete in order
		const int lc = hf * 80 + 4 * grp;  // tile column of the lane's first value
		const int col = n0 + lc, c0 = col & ~15;
		const int32_t* pf = prm + 3 * lc;
		const v4i p0 = *(const v4i*)pf, p1 = *(const v4i*)(pf + 4), p2 = *(const v4i*)(pf + 8);
		// parameters of columns lc .. lc + 3: (p0.x p0.y p0.z) (p0.w p1.x p1.y) (p1.z p1.w p2.x) (p2.y p2.z p2.w)
		const FoldConsts fc0 = fold_consts(p0[0], p0[1], p0[2]), fc1 = fold_consts(p0[3], p1[0], p1[1]);
		const FoldConsts fc2 = fold_consts(p1[2], p1[3], p2[0]), fc3 = fold_consts(p2[1], p2[2], p2[3]);
		const int si = (e.nseg > 1 && c0 >= e.seg[0].n_end) ? ((e.nseg > 2 && c0 >= e.seg[1].n_end) ? 2 : 1) : 0;
#define SSLM_SEG_FIELD(f) (si == 0 ? e.seg[0].f : (si == 1 ? e.seg[1].f : e.seg[2].f))
		const int nbeg = SSLM_SEG_FIELD(n_begin), ld = SSLM_SEG_FIELD(ld_out);
		int32_t* sout = (int32_t*)SSLM_SEG_FIELD(out);
		uint32_t* smax = SSLM_SEG_FIELD(maxpart);
#undef SSLM_SEG_FIELD
		const bool col_ok = rp < RST && col < g.N;
		int32_t* op = sout + (size_t)rowb * ld + (col - nbeg);
		uint32_t* mp = smax ? smax + (size_t)(c0 >> 4) * kPartLd + rowb : nullptr;
		// all the half's reads first (rows up to 66 of the last wave's slab stay inside the
		// parameter block after it; rows past 63 are read, never used)
		const int32_t* sp = slab + rp * LDW + 4 * grp;
		v4i av[RITER];
#pragma unroll
		for (int k = 0; k < RITER; ++k) av[k] = *(const v4i*)(sp + k * RST * LDW);
#pragma unroll
		for (int k = 0; k < RITER; ++k) {
			if (k * RST + RST > 64 && rp >= 64 - k * RST) break;  // past the slab (quad-uniform)
			const v4i a = av[k];
			v4i o;
			o[0] = fold_bounded(a[0], fc0);
			o[1] = fold_bounded(a[1], fc1);
			o[2] = fold_bounded(a[2], fc2);
			o[3] = fold_bounded(a[3], fc3);
			const bool ok = col_ok && rowb + k * RST < g.M;
			if (ok) *(v4i*)(op + (size_t)k * RST * ld) = o;
			uint32_t mx = 0;
#pragma unroll
			for (int q = 0; q < 4; ++q) mx = max(mx, o[q] < 0 ? 0u - (uint32_t)o[q] : (uint32_t)o[q]);
			if (!ok) mx = 0;
			// quad max (quad_perm [1,0,3,2] then [2,3,0,1]): the 4 lanes of one 16-column tile
			uint32_t w2 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mx, 0xb1, 0xf, 0xf, false);
			mx = max(mx, w2);
			w2 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mx, 0x4e, 0xf, 0xf, false);
			mx = max(mx, w2);
			if ((lane & 3) == 0 && ok && mp) mp[k * RST] = mx;
		}
	}
}

// ------------------------------------------------------------------------------------------
// Narrow prefill GEMM (M > 64, few 256 x 128 tiles): 64 x 64 block tiles over the whole K, raw
// int32 output (one plane; the consuming row kernel applies the epilogue, RawIn).  The
// projections whose N is a few thousand columns (q|k|v, o, down) have too few 256 x 128 tiles
// to fill 256 CUs; the K-split alternative writes one int32 plane per split, several times the
// output, which then is read back.  Small tiles fill the chip with the whole K per block and
// write the output once.
// Block: 4 waves, wave w owns the 32 x 32 sub-tile (w / 2, w % 2) as two v_mfma_i32_32x32x32_i8
// accumulators (even and odd 32-deep steps, two independent chains).  Operands go global ->
// LDS directly through NN = 4 stages of 128-deep K steps (16 KB each, XOR-swizzled rows as in
// lds_chunk); two blocks per CU overlap one's loads and epilogue with the other's MFMAs.
// Loads are unconditional (rows past M or N read a clamped valid row; their products land only in
// discarded outputs) and K is a multiple of 128.
// ------------------------------------------------------------------------------------------
constexpr int kNarrowTile = 64, kNarrowStages = 4, kNarrowMaxK = 4096;

// lgkmcnt(0) that the two fragments pass through
__device__ __forceinline__ void lgkm_wait2(v4i& a, v4i& b) { asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b)); }

__global__ __launch_bounds__(256, 2) void k_gemm_narrow(GemmArgs g) {
	constexpr int NN = kNarrowStages, T = kNarrowTile;
	constexpr int STAGE = 2 * T * kPStride;  // A rows then W rows, 128 bytes each
	constexpr int CPT = STAGE / 1024 / 4;    // 1 KB direct loads per wave per stage
	__shared__ __attribute__((aligned(1024))) int8_t smem[NN * STAGE];
	const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
	const int tiles_m = (g.M + T - 1) / T;
	const int B = gridDim.x;
	// XCD-aware order (workgroups go round-robin over the 8 XCDs): tiles that share W rows
	// (same column block) land in one XCD's L2
	const int vb = B % 8 == 0 ? (int)(blockIdx.x % 8) * (B / 8) + (int)(blockIdx.x / 8) : (int)blockIdx.x;
	const int m0 = (vb % tiles_m) * T, n0 = (vb / tiles_m) * T;
	const int S = g.K / kPBK;
	const int8_t* src[CPT];
#pragma unroll
	for (int j = 0; j < CPT; ++j) {
		const int slot = (wave * CPT + j) * 64 + lane;
		const int row = slot >> 3, pc = slot & 7;
		const int q = pc ^ ((row >> 1) & 7);
		if (row < T) src[j] = g.a + (size_t)min(m0 + row, g.M - 1) * g.lda + q * 16;
		else src[j] = g.w + (size_t)min(n0 + row - T, g.N - 1) * g.K + q * 16;
	}
	auto issue = [&](int st, int t) {  // past the last step the last is fetched again (never read)
		const size_t kb = (size_t)min(t, S - 1) * kPBK;
#pragma unroll
		for (int j = 0; j < CPT; ++j)
			__builtin_amdgcn_global_load_lds((const void*)(src[j] + kb),
			                                 (__attribute__((address_space(3))) void*)(smem + st * STAGE + (wave * CPT + j) * 1024),
			                                 16, 0, 0);
	};
	const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
	const uint32_t lds0 = (uint32_t)(size_t)(__attribute__((address_space(3))) int8_t*)smem;
	uint32_t aoff[4], boff[4];  // the lane's 16-byte chunk of each 32-deep step
#pragma unroll
	for (int ks = 0; ks < 4; ++ks) {
		aoff[ks] = lds0 + lds_chunk(wm + (lane & 31), 2 * ks + (lane >> 5));
		boff[ks] = lds0 + lds_chunk(T + wn + (lane & 31), 2 * ks + (lane >> 5));
	}
	v16i acc0, acc1;
#pragma unroll
	for (int v = 0; v < 16; ++v) acc0[v] = acc1[v] = 0;
#pragma unroll
	for (int s0 = 0; s0 < NN - 1; ++s0) issue(s0, s0);
	for (int t = 0; t < S; ++t) {
		wait_vmcnt<(NN - 2) * CPT>();  // own loads of step t have landed
		// bare barrier: every wave's loads of step t have landed and every wave is done with step
		// t - 1, whose stage takes step t + NN - 1 (a __syncthreads() fence would drain the loads)
		__builtin_amdgcn_s_barrier();
		issue((t + NN - 1) % NN, t + NN - 1);
		const uint32_t so = (uint32_t)((t % NN) * STAGE);
		v4i a0 = lds_read16<0>(aoff[0] + so), b0 = lds_read16<0>(boff[0] + so);
		v4i a1 = lds_read16<0>(aoff[1] + so), b1 = lds_read16<0>(boff[1] + so);
		v4i a2 = lds_read16<0>(aoff[2] + so), b2 = lds_read16<0>(boff[2] + so);
		v4i a3 = lds_read16<0>(aoff[3] + so), b3 = lds_read16<0>(boff[3] + so);
		lgkm_wait2(a0, b0);
		lgkm_wait2(a1, b1);
		lgkm_wait2(a2, b2);
		lgkm_wait2(a3, b3);
		acc0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, b0, acc0, 0, 0, 0);
		acc1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, b1, acc1, 0, 0, 0);
		acc0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a2, b2, acc0, 0, 0, 0);
		acc1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a3, b3, acc1, 0, 0, 0);
	}
	wait_vmcnt<0>();  // the trailing (clamped) loads land before the block ends
	// 32x32 layout: lane holds column lane % 32, rows 8 (v / 4) + 4 (lane / 32) + v % 4
	int32_t* out = g.epi.raw_out;
	const int col = n0 + wn + (lane & 31);
	if (col < g.N) {
#pragma unroll
		for (int v = 0; v < 16; ++v) {
			const int row = m0 + wm + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
			if (row < g.M) out[(size_t)row * g.N + col] = acc0[v] + acc1[v];
		}
	}
}

// ------------------------------------------------------------------------------------------
// row kernels (one block per token)
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
	for (int i = threadIdx.x; i < H; i += kRowBlock) out[i] = requant_code_f(row[i], requant_factor(plan.r, plan.s));
	if (threadIdx.x == 0) out_scale[scale_idx[t]] = plan.out;
}

// ------------------------------------------------------------------------------------------
// Latency-oriented row kernels.  A decode row is short (H or I elements) and its funnel is a
// chain of dependent steps (max -> scale plan -> codes -> max -> ...), so these kernels are
// shaped for latency, not bandwidth: every independent global load is issued at entry, the row
// stays in registers (EPT values per thread, element i = threadIdx.x + k * BS), each block
// reduction costs a single barrier (every call site owns its LDS slots), and the scalar scale
// plans are evaluated redundantly by all threads instead of by one thread and a broadcast.
// A slot's status is read once by thread 0 and tested after the first barrier, so the whole
// block leaves together.
// ------------------------------------------------------------------------------------------
// A block reduction's result is the same in every lane; saying so (readfirstlane) lets the
// compiler keep it, and the scalar scale plans computed from it, in scalar registers.
__device__ __forceinline__ uint64_t uni_u64(uint64_t v) {
	const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
	const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
	return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ int64_t uni_i64(int64_t v) { return (int64_t)uni_u64((uint64_t)v); }

// 32-bit wave reductions: a 16-lane rotate butterfly (DPP) leaves every lane with its row's
// result, and the four row results are read as scalars -- the value comes back wave-uniform.
__device__ __forceinline__ uint32_t wave_max32(uint32_t v) {
	v = dpp_max16(v);
	const uint32_t a = __builtin_amdgcn_readlane(v, 0), b = __builtin_amdgcn_readlane(v, 16);
	const uint32_t c = __builtin_amdgcn_readlane(v, 32), d = __builtin_amdgcn_readlane(v, 48);
	return max(max(a, b), max(c, d));
}

__device__ __forceinline__ int32_t wave_sum32(int32_t v) {
	v += __builtin_amdgcn_update_dpp(0, v, 0x128, 0xf, 0xf, false);  // row_ror:8
	v += __builtin_amdgcn_update_dpp(0, v, 0x124, 0xf, 0xf, false);  // row_ror:4
	v += __builtin_amdgcn_update_dpp(0, v, 0x122, 0xf, 0xf, false);  // row_ror:2
	v += __builtin_amdgcn_update_dpp(0, v, 0x121, 0xf, 0xf, false);  // row_ror:1
	return __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16) + __builtin_amdgcn_readlane(v, 32) +
	       __builtin_amdgcn_readlane(v, 48);
}

// block reductions with one barrier; each call site owns its LDS slots (BS / 64 entries)
template <int BS>
__device__ __forceinline__ uint32_t blk_max32(uint32_t v, uint32_t* slots) {
	v = wave_max32(v);
	if ((threadIdx.x & 63) == 0) slots[threadIdx.x >> 6] = v;
	__syncthreads();
	uint32_t r = slots[0];
#pragma unroll
	for (int i = 1; i < BS / 64; ++i) r = max(r, slots[i]);
	return __builtin_amdgcn_readfirstlane(r);
}

// two maxima, one barrier; `slots` holds 2 * BS / 64 entries
template <int BS>
__device__ __forceinline__ void blk_max32x2(uint32_t& x, uint32_t& y, uint32_t* slots) {
	x = wave_max32(x);
	y = wave_max32(y);
	if ((threadIdx.x & 63) == 0) {
		slots[threadIdx.x >> 6] = x;
		slots[BS / 64 + (threadIdx.x >> 6)] = y;
	}
	__syncthreads();
	x = slots[0];
	y = slots[BS / 64];
#pragma unroll
	for (int i = 1; i < BS / 64; ++i) {
		x = max(x, slots[i]);
		y = max(y, slots[BS / 64 + i]);
	}
	x = __builtin_amdgcn_readfirstlane(x);
	y = __builtin_amdgcn_readfirstlane(y);
}

template <int BS>
__device__ __forceinline__ int32_t blk_sum32(int32_t v, int32_t* slots) {
	v = wave_sum32(v);
	if ((threadIdx.x & 63) == 0) slots[threadIdx.x >> 6] = v;
	__syncthreads();
	int32_t r = 0;
#pragma unroll
	for (int i = 0; i < BS / 64; ++i) r += slots[i];
	return __builtin_amdgcn_readfirstlane(r);
}

// this thread's share of the max over tiles [tile0, tile0 + ntiles) of a per-(tile, token)
// partial array (32-bit); combine across the block with blk_max32
// Elements threadIdx.x + k * BS (k < EPT) of a row of n >= 1 elements, 0 beyond n.  The loads
// are unconditional (clamped indices): a load under a per-lane branch makes the compiler wait
// for it before the branch joins, so guarded loads cost one memory round trip each.
template <int BS, int EPT, typename T>
__device__ __forceinline__ void load_row_raw(const T* row, int n, T (&v)[EPT]) {
#pragma unroll
	for (int k = 0; k < EPT; ++k) v[k] = row[min((int)threadIdx.x + k * BS, n - 1)];
}
template <int BS, int EPT, typename T>
__device__ __forceinline__ void row_take(const T (&v)[EPT], int n, int32_t (&out)[EPT]) {
#pragma unroll
	for (int k = 0; k < EPT; ++k) out[k] = (int)threadIdx.x + k * BS < n ? (int32_t)v[k] : 0;
}
template <int BS, int EPT, typename T>
__device__ __forceinline__ void load_row(const T* row, int n, int32_t (&out)[EPT]) {
	T v[EPT];
	load_row_raw<BS>(row, n, v);
	row_take<BS>(v, n, out);
}

// The maximum over per-tile partial maxima [tile0, tile0 + ntiles) of token t, for ntiles <= PER * BS,
// as straight-line code: every thread issues its PER loads at once from clamped indices, so the
// partials cost one memory round trip rather than one per loop iteration
template <int BS, int PER>
__device__ __forceinline__ uint32_t part_max32_fixed(const uint32_t* part, int tile0, int ntiles, int t) {
	uint32_t v[PER];
#pragma unroll
	for (int k = 0; k < PER; ++k) v[k] = part[(size_t)(tile0 + min((int)threadIdx.x + k * BS, max(ntiles - 1, 0))) * kPartLd + t];
	uint32_t m = 0;
#pragma unroll
	for (int k = 0; k < PER; ++k) m = max(m, (int)threadIdx.x + k * BS < ntiles ? v[k] : 0u);
	return m;
}

template <int BS>
__device__ __forceinline__ uint64_t blk_max(uint64_t v, uint64_t* slots) {
	v = wave_max_u64(v);
	if ((threadIdx.x & 63) == 0) slots[threadIdx.x >> 6] = v;
	__syncthreads();
	uint64_t r = slots[0];
#pragma unroll
	for (int i = 1; i < BS / 64; ++i) r = slots[i] > r ? slots[i] : r;
	return uni_u64(r);
}

template <int BS>
__device__ __forceinline__ int64_t blk_max_i64(int64_t v, int64_t* slots) {
	v = wave_max_i64(v);
	if ((threadIdx.x & 63) == 0) slots[threadIdx.x >> 6] = v;
	__syncthreads();
	int64_t r = slots[0];
#pragma unroll
	for (int i = 1; i < BS / 64; ++i) r = slots[i] > r ? slots[i] : r;
	return uni_i64(r);
}


// N elements (columns j[k] of segment `si`) of token t of a raw split-K projection with the
// segment's epilogue applied (RawIn).  Every load -- all split planes, fold triples and biases
// -- is issued before the first use, in straight-line code, so the row pays one memory round
// trip.  Columns with live[k] false read a valid column and return 0.  Returns false when a bias
// reconcile refused its product (epi_value's rule).
template <int N, int S>
__device__ __forceinline__ bool raw_row(const RawIn& r, int si, int M, int t, const int (&j)[N], const bool (&live)[N],
                                        int64_t (&v)[N]) {
	const Segment& sg = r.epi.seg[si];
	const size_t plane = (size_t)M * r.ld;
	const int32_t* row = r.part + (size_t)t * r.ld;
	int32_t jj[N];
	uint32_t acc[N];
	int32_t f0[N], f1[N], f2[N];
#pragma unroll
	for (int k = 0; k < N; ++k) {
		const int jc = live[k] ? j[k] : sg.n_begin;
		jj[k] = jc - sg.n_begin;
		acc[k] = 0;
#pragma unroll
		for (int s2 = 0; s2 < S; ++s2) {  // clamped plane index: no branch, no extra round trip
			const uint32_t x = (uint32_t)row[(size_t)(S == 1 ? 0 : min(s2, r.splits - 1)) * plane + jc];
			acc[k] += (S == 1 || s2 < r.splits) ? x : 0u;  // the true sum fits int32; partials wrap harmlessly
		}
		const int32_t* f = sg.fold + 3 * jj[k];
		f0[k] = f[0];
		f1[k] = f[1];
		f2[k] = f[2];
	}
	int64_t bias[N];
	int64_t rcp = 0, ein = 0;
	if (sg.bias) {
#pragma unroll
		for (int k = 0; k < N; ++k) bias[k] = sg.bias[jj[k]];
		rcp = r.epi.in_recip[t];
		ein = r.epi.in_scale[t].e;
	}
	bool ok = true;
#pragma unroll
	for (int k = 0; k < N; ++k) {
		v[k] = apply_fold((int64_t)(int32_t)acc[k], f0[k], f1[k], f2[k]);
		if (sg.lora_b) {
			v[k] += lora_delta(sg, r.epi.rank, t, jj[k]);
		}
		if (sg.bias) {
			int64_t term;
			if (bias_term(bias[k], rcp, ein, v[k], &term)) v[k] += term;
			else if (live[k]) ok = false;
		}
		if (!live[k]) v[k] = 0;
	}
	return ok;
}

constexpr int32_t kSkipped = -1;  // the slot had already failed: nothing written, no status

// forward_sites.cpp:410-459 -- the RMSNorm site body on a register-resident row of codes `h`
// (zero beyond H) with gains `g`.  `prior` (LDS, or null) is the slot status read before entry.
template <int BS, int EPT>
__device__ __forceinline__ int32_t rmsnorm_regs(const int32_t (&h)[EPT], const int32_t (&g)[EPT], int H, Scale site,
                                                int8_t* out, Scale* out_scale, int64_t* out_recip, int32_t* s_sum,
                                                uint32_t* s_max, const int32_t* prior) {
	int32_t ss = 0;  // sum of squared int8 codes: < 2^14 * H, exact in int32
#pragma unroll
	for (int k = 0; k < EPT; ++k) ss += h[k] * h[k];
	ss = blk_sum32<BS>(ss, s_sum);
	KT(10);
	if (prior && *prior != 0) return kSkipped;
	int64_t root = isqrt_fast(div_floor_pos((int64_t)ss << 32, (int64_t)H));
	root = root > 1 ? root : 1;
	// floor((v << 32) / root) per element from one shared reciprocal (root < 2^23)
	const double rd = (double)root, inv = 1.0 / rd;
	KT(11);
	int64_t w[EPT];
	uint32_t mx = 0;
#pragma unroll
	for (int k = 0; k < EPT; ++k) {
		w[k] = norm_fd(h[k], rd, inv) * (int64_t)g[k];
		mx = max(mx, sat_abs_u32(w[k]));
	}
	mx = blk_max32<BS>(mx, s_max);
	KT(12);
	FunnelPlan plan;
	const int32_t st = funnel_plan(mx, nullptr, 0, site, &plan);
	if (st != kOk) return st;
	KT(13);
#pragma unroll
	for (int k = 0; k < EPT; ++k) {
		const int i = threadIdx.x + k * BS;
		if (i < H) out[i] = requant_code_f(w[k], requant_factor(plan.r, plan.s));
	}
	if (threadIdx.x == 0) {
		*out_scale = plan.out;
		if (out_recip) *out_recip = fits_i32(plan.out.m) ? reciprocal_fast(plan.out.m) : 0;
	}
	return kOk;
}

template <int BS, int EPT>
__global__ __launch_bounds__(BS) void k_rmsnorm(sslm_launch::RowNormArgs a, int H, const TokenInfo* tok,
                                              int32_t* status, int32_t layer) {
	__shared__ int32_t s_sum[BS / 64];
	__shared__ uint32_t s_max[BS / 64];
	__shared__ int32_t s_st;
	const int t = blockIdx.x;
	const int slot = tok[t].slot;
	const int8_t* hrow = a.in_codes + (size_t)a.in_idx[t] * a.ld_in;
	int32_t h[EPT], g[EPT];
	load_row<BS>(hrow, H, h);
	load_row<BS>(a.gain, H, g);
	if (threadIdx.x == 0) s_st = status[slot];
	const int32_t st = rmsnorm_regs<BS, EPT>(h, g, H, a.site, a.out + (size_t)t * H, &a.out_scale[t],
	                                         a.out_recip ? &a.out_recip[t] : nullptr, s_sum, s_max, &s_st);
	if (threadIdx.x == 0 && st > 0) set_status(status, slot, layer, st);
}

// q funnel + RoPE(q); K/V landing, RoPE(K), KV write (forward_sites.cpp:1281-1418, :1748-1787).
// The K/V landing does not depend on the q funnel, so it is computed while the q maximum is
// reduced.  Up to 2 K (and 2 V) pairs per thread: NKV * D <= 4 * BS.
template <int BS, int EQ, int RS>
__global__ __launch_bounds__(BS) void k_qkv_post(sslm_launch::QkvPostArgs a) {
	__shared__ uint32_t s_red[BS / 64];
	__shared__ int32_t s_st;
	const int t = xcd_row(blockIdx.x, gridDim.x);
	const TokenInfo ti = a.tok[t];
	const Scale ns = a.in_scale[t];
	const int H = a.H, D = a.D, pairs = D / 2;
	const int KVH = a.NKV * D;
	const int64_t pos = ti.pos;
	const bool pos_ok = pos >= 0 && pos < a.cap;
	const int64_t* cs = a.rope_cos + (pos_ok ? pos : 0) * pairs;
	const int64_t* sn = a.rope_sin + (pos_ok ? pos : 0) * pairs;
	// q pair values
	int2 qv[EQ];
	uint32_t qmx = 0;
	if (RS > 0) {
		int j[2 * EQ];
		bool live[2 * EQ];
		int64_t v[2 * EQ];
#pragma unroll
		for (int k = 0; k < EQ; ++k) {
			const int p = threadIdx.x + k * BS;
			j[2 * k] = 2 * p;
			j[2 * k + 1] = 2 * p + 1;
			live[2 * k] = live[2 * k + 1] = p < H / 2;
		}
		const bool ok = raw_row<2 * EQ, RS>(a.raw, 0, a.M, t, j, live, v);
#pragma unroll
		for (int k = 0; k < EQ; ++k) {
			qv[k] = make_int2(sat_i32(v[2 * k]), sat_i32(v[2 * k + 1]));
			qmx = max(qmx, max(sat_abs_u32(v[2 * k]), sat_abs_u32(v[2 * k + 1])));
		}
		if (!ok) qmx = kBad32;
	} else {
		const int2* qf = (const int2*)(a.q_f + (size_t)t * H);
		int2 qr[EQ];
#pragma unroll
		for (int k = 0; k < EQ; ++k) qr[k] = qf[min((int)threadIdx.x + k * BS, H / 2 - 1)];  // clamped: no per-lane branch
#pragma unroll
		for (int k = 0; k < EQ; ++k) qv[k] = (int)threadIdx.x + k * BS < H / 2 ? qr[k] : make_int2(0, 0);
		qmx = part_max32_fixed<BS, (2 * EQ + 15) / 16>(a.q_maxpart, 0, H / 16, t);  // H <= 2 * EQ * BS
	}
	if (threadIdx.x == 0) s_st = a.status[ti.slot];
	// K/V landing (LandingRescale at the normed scale, per kv head) and RoPE(K)
	const int64_t* kv = RS > 0 ? nullptr : a.kv_f + (size_t)t * 2 * KVH;
	int8_t kq[2][2], vq[2][2];
	uint64_t sat = 0;
	int64_t rk[4], rv[4];
	if (RS > 0) {
		int jk[4], jv[4];
		bool live[4];
#pragma unroll
		for (int k = 0; k < 2; ++k) {
			const int p = threadIdx.x + k * BS;
			jk[2 * k] = H + 2 * p;
			jk[2 * k + 1] = H + 2 * p + 1;
			jv[2 * k] = H + KVH + 2 * p;
			jv[2 * k + 1] = H + KVH + 2 * p + 1;
			live[2 * k] = live[2 * k + 1] = p < KVH / 2;
		}
		const bool okk = raw_row<4, RS>(a.raw, 1, a.M, t, jk, live, rk);
		const bool okv = raw_row<4, RS>(a.raw, 2, a.M, t, jv, live, rv);
		if (!(okk && okv)) qmx = kBad32;
	}
#pragma unroll
	for (int k = 0; k < 2; ++k) {
		const int p = threadIdx.x + k * BS;
		if (p < KVH / 2) {  // (an out-of-range position is refused below; its values are unused)
			const int hd = (2 * p) / D;
			const int i = p % pairs;
			longlong2 kk, vv;
			if (RS > 0) {
				kk = make_longlong2(rk[2 * k], rk[2 * k + 1]);
				vv = make_longlong2(rv[2 * k], rv[2 * k + 1]);
			} else {
				kk = ((const longlong2*)kv)[p];
				vv = ((const longlong2*)(kv + KVH))[p];
			}
			const int64_t k_e = composed_exponent(ns.e, a.e_t_k[hd]);
			const int64_t v_e = composed_exponent(ns.e, a.e_t_v[hd]);
			const int64_t rtk = a.r_t_k[hd], rtv = a.r_t_v[hd];
			bool c0, c1, c2, c3, x0;
			const int64_t k0 = clamp_code(landing_rescale(kk.x, ns.m, rtk, k_e, &c0, &x0));
			const int64_t k1 = clamp_code(landing_rescale(kk.y, ns.m, rtk, k_e, &c1, &x0));
			int64_t xr, yr;
			rope_pair((int32_t)k0, (int32_t)k1, (int32_t)cs[i], (int32_t)sn[i], &xr, &yr);
			kq[k][0] = (int8_t)clamp_code(xr);
			kq[k][1] = (int8_t)clamp_code(yr);
			vq[k][0] = (int8_t)clamp_code(landing_rescale(vv.x, ns.m, rtv, v_e, &c2, &x0));
			vq[k][1] = (int8_t)clamp_code(landing_rescale(vv.y, ns.m, rtv, v_e, &c3, &x0));
			sat += (uint64_t)c0 + (uint64_t)c1 + (uint64_t)c2 + (uint64_t)c3;
		}
	}
	qmx = blk_max32<BS>(qmx, s_red);
	if (s_st != 0) return;
	FunnelPlan plan;
	int32_t st = qmx == kBad32 ? kBiasReconcileProductOutOfDomain : funnel_plan(qmx, &ns, 1, a.q_site, &plan);
	if (st == kOk && !pos_ok) st = kPositionOverCap;
	if (st != kOk) {
		if (threadIdx.x == 0) set_status(a.status, ti.slot, a.layer, st);
		return;
	}
	// q: codes of pair (2i, 2i+1), rotated, clamped
	char2* qo = (char2*)(a.q_rot + (size_t)t * H);
#pragma unroll
	for (int k = 0; k < EQ; ++k) {
		const int p = threadIdx.x + k * BS;
		if (p < H / 2) {
			const int i = p % pairs;
			const int32_t x = requant_code_f(qv[k].x, requant_factor(plan.r, plan.s));
			const int32_t y = requant_code_f(qv[k].y, requant_factor(plan.r, plan.s));
			int64_t xr, yr;
			rope_pair(x, y, (int32_t)cs[i], (int32_t)sn[i], &xr, &yr);
			qo[p] = make_char2((char)clamp_code(xr), (char)clamp_code(yr));
		}
	}
	if (threadIdx.x == 0) a.q_scale[t] = plan.out;
	if (a.kv_stage) {  // prefill span: staged until every token's q funnel has passed
		int8_t* row = a.kv_stage + (size_t)t * 2 * KVH;
#pragma unroll
		for (int k = 0; k < 2; ++k) {
			const int p = threadIdx.x + k * BS;
			if (p < KVH / 2) {
				*(char2*)(row + 2 * p) = make_char2(kq[k][0], kq[k][1]);
				*(char2*)(row + KVH + 2 * p) = make_char2(vq[k][0], vq[k][1]);
			}
		}
		sat = wave_sum_i64((int64_t)sat);
		if ((threadIdx.x & 63) == 0 && sat) atomicAdd(&a.sat_stage[t], (uint32_t)sat);
		return;
	}
	int8_t* blk = a.kv_pool + (int64_t)ti.block * a.block_bytes;
	const int64_t half = a.cap * (int64_t)KVH;
	int8_t* kstore = blk + (int64_t)a.layer * half * 2;
	int8_t* vstore = kstore + half;
#pragma unroll
	for (int k = 0; k < 2; ++k) {
		const int p = threadIdx.x + k * BS;
		if (p < KVH / 2) {
			const int hd = (2 * p) / D;
			const int i = p % pairs;
			const int64_t off = ((int64_t)hd * a.cap + pos) * D + 2 * i;
			*(char2*)(kstore + off) = make_char2(kq[k][0], kq[k][1]);
			*(char2*)(vstore + off) = make_char2(vq[k][0], vq[k][1]);
		}
	}
	sat = wave_sum_i64((int64_t)sat);
	if ((threadIdx.x & 63) == 0 && sat) atomicAdd(&a.sat[ti.slot], (unsigned long long)sat);
}

// Looped form of k_slot_state_copy for rows or K/V spans past its fixed per-thread counts.
__global__ __launch_bounds__(256) void k_slot_state_copy_any(sslm_launch::SlotCopyArgs a, int restore) {
	const TokenInfo ti = a.tok[blockIdx.x];
	const int64_t slot = ti.slot;
	int8_t* live = a.codes + slot * a.H;
	int8_t* snap = a.snap_codes + slot * a.H;
	for (int i = threadIdx.x; i < a.H; i += blockDim.x) {
		if (restore) live[i] = snap[i];
		else snap[i] = live[i];
	}
	if (threadIdx.x == 0) {
		if (restore) {
			a.scale[slot] = a.snap_scale[slot];
			a.sat[slot] = a.snap_sat[slot];
		} else {
			a.snap_scale[slot] = a.scale[slot];
			a.snap_sat[slot] = a.sat[slot];
		}
	}
	const int KVH = a.NKV * a.D, per_layer = 2 * KVH;
	if (ti.pos < 0 || ti.pos >= a.cap) return;
	const int64_t half = a.cap * (int64_t)KVH;
	int8_t* blk = a.kv_pool + (int64_t)ti.block * a.block_bytes;
	int8_t* srow = a.snap_kv + slot * a.snap_kv_ld;
	for (int c = threadIdx.x; c < (a.l1 - a.l0) * per_layer / 16; c += blockDim.x) {
		const int e = c * 16, l = a.l0 + e / per_layer, r = e % per_layer;
		const int kvsel = r >= KVH, hd = (r - kvsel * KVH) / a.D, d = (r - kvsel * KVH) % a.D;
		int4* kvp = (int4*)(blk + (int64_t)l * half * 2 + kvsel * half + ((int64_t)hd * a.cap + ti.pos) * a.D + d);
		int4* sp = (int4*)(srow + (int64_t)l * per_layer + r);
		if (restore) *kvp = *sp;
		else *sp = *kvp;
	}
}

// Every load of the block is issued before the first store (16-byte vectors, clamped indices, a
// fixed unrolled count per thread), so the copy is one memory round trip rather than one per
// loop iteration.
constexpr int kSnapKvPer = 8;  // K/V chunks of 16 bytes per thread: (l1 - l0) 2 NKV D <= 32 KB

__global__ __launch_bounds__(256) void k_slot_state_copy(sslm_launch::SlotCopyArgs a, int restore) {
	const TokenInfo ti = a.tok[blockIdx.x];
	const int64_t slot = ti.slot;
	int8_t* live = a.codes + slot * a.H;
	int8_t* snap = a.snap_codes + slot * a.H;
	const int8_t* csrc = restore ? snap : live;
	int8_t* cdst = restore ? live : snap;
	// the stream row: H / 16 vectors (H is a multiple of 16), one per thread
	const int nv = a.H / 16, vi = min((int)threadIdx.x, nv - 1);
	const v4i cv = load16(csrc + vi * 16);
	const Scale sc = restore ? a.snap_scale[slot] : a.scale[slot];
	const unsigned long long sv = restore ? a.snap_sat[slot] : a.sat[slot];
	// the K and V rows of layers [l0, l1) at the token's position
	const int KVH = a.NKV * a.D, per_layer = 2 * KVH;
	const bool pos_ok = ti.pos >= 0 && ti.pos < a.cap;
	const int64_t pos = pos_ok ? ti.pos : 0;
	const int64_t half = a.cap * (int64_t)KVH;
	int8_t* blk = a.kv_pool + (int64_t)ti.block * a.block_bytes;
	int8_t* srow = a.snap_kv + slot * a.snap_kv_ld;
	const int nc = (a.l1 - a.l0) * per_layer / 16;
	// vector loads and stores (ext_vector_type) keep kv[] in registers
	int8_t* kvp[kSnapKvPer];
	int8_t* sp[kSnapKvPer];
	v4i kv[kSnapKvPer];
#pragma unroll
	for (int k = 0; k < kSnapKvPer; ++k) {
		const int c = min((int)threadIdx.x + k * 256, nc - 1);
		const int e = c * 16, l = a.l0 + e / per_layer, r = e % per_layer;
		const int kvsel = r >= KVH, hd = (r - kvsel * KVH) / a.D, d = (r - kvsel * KVH) % a.D;
		kvp[k] = blk + (int64_t)l * half * 2 + kvsel * half + ((int64_t)hd * a.cap + pos) * a.D + d;
		sp[k] = srow + (int64_t)l * per_layer + r;
		kv[k] = load16(restore ? sp[k] : kvp[k]);
	}
	if ((int)threadIdx.x < nv) *(v4i*)(cdst + threadIdx.x * 16) = cv;
	if (threadIdx.x == 0) {
		if (restore) {
			a.scale[slot] = sc;
			a.sat[slot] = sv;
		} else {
			a.snap_scale[slot] = sc;
			a.snap_sat[slot] = sv;
		}
	}
	if (!pos_ok) return;
#pragma unroll
	for (int k = 0; k < kSnapKvPer; ++k) {
		if ((int)threadIdx.x + k * 256 < nc) {
			*(v4i*)(restore ? kvp[k] : sp[k]) = kv[k];
		}
	}
}

// One block per token of a prefill span: the staged K/V row into the pool (16 bytes per
// thread), the token's clamp count into the slot's counter.
__global__ __launch_bounds__(256) void k_kv_commit(sslm_launch::QkvPostArgs a) {
	__shared__ int32_t s_st;
	const int t = blockIdx.x;
	const TokenInfo ti = a.tok[t];
	const int D = a.D, KVH = a.NKV * D;
	if (threadIdx.x == 0) {
		s_st = a.status[ti.slot];
		const uint32_t sat = a.sat_stage[t];
		a.sat_stage[t] = 0;
		if (s_st == 0 && sat) atomicAdd(&a.sat[ti.slot], (unsigned long long)sat);
	}
	__syncthreads();
	if (s_st != 0) return;
	const int8_t* row = a.kv_stage + (size_t)t * 2 * KVH;
	const int64_t half = a.cap * (int64_t)KVH;
	int8_t* kstore = a.kv_pool + (int64_t)ti.block * a.block_bytes + (int64_t)a.layer * half * 2;
	for (int c = threadIdx.x; c < 2 * KVH / 16; c += blockDim.x) {
		const int e = c * 16;              // element of [K heads | V heads]
		const int kvsel = e >= KVH;        // 0: K, 1: V
		const int hd = (e - kvsel * KVH) / D, d = (e - kvsel * KVH) % D;
		*(int4*)(kstore + kvsel * half + ((int64_t)hd * a.cap + ti.pos) * D + d) = *(const int4*)(row + e);
	}
}

// funnel over an int32 fold-output row (checked_chain_funnel.cpp:257-364)
template <int BS, int EPT>
__global__ __launch_bounds__(BS) void k_funnel(sslm_launch::FunnelArgs a) {
	__shared__ uint32_t s_m[BS / 64];
	__shared__ int32_t s_st;
	const int t = xcd_row(blockIdx.x, gridDim.x), N = a.N;
	const int slot = a.tok[t].slot;
	const int32_t* frow = a.f + (size_t)t * a.ld_f;
	// the maxima, scales and status words first, then the row: the plan needs only the former, so
	// the block reduction and the plan run while the row is in flight
	uint32_t mx = part_max32_fixed<BS, (EPT + 15) / 16>(a.maxpart, 0, a.ntiles, t);  // ntiles <= N / 16 + 1
	Scale inc{0, 0};
	if (a.incoming) inc = a.incoming[t];
	const int32_t st0 = a.status[slot];
	const int32_t hs0 = (a.head_status ? a.head_status : a.status)[slot];
	const int32_t hs = a.head_status ? hs0 : kHeadStatusNone;  // the first refusing head of the attention
	int32_t fv[EPT];
	load_row_raw<BS>(frow, N, fv);
	asm volatile("" ::"s"(st0), "s"(hs0));  // both status loads issued together, ahead of the branch
	if (threadIdx.x == 0) {
		// each branch stores its own value: through a join, the rare path's re-read would make
		// the common path wait for every load of wave 0 (its row included) before the reduction
		if (hs != kHeadStatusNone) {  // rare: resolve the attention's refusal into the status
			set_status(a.status, slot, a.layer, hs & 0xff);
			a.head_status[slot] = kHeadStatusNone;
			s_st = a.status[slot];
			asm volatile("" ::: "memory");
		} else {
			s_st = st0;
		}
	}
	mx = blk_max32<BS>(mx, s_m);
	if (s_st != 0) return;
	FunnelPlan plan;
	const int32_t st = funnel_plan(mx, a.incoming ? &inc : nullptr, a.incoming ? 1 : 0, a.site, &plan);
	if (st != kOk) {
		if (threadIdx.x == 0) set_status(a.status, slot, a.layer, st);
		return;
	}
	int32_t f[EPT];
	row_take<BS>(fv, N, f);
	int8_t* out = a.out + (size_t)t * N;
#pragma unroll
	for (int k = 0; k < EPT; ++k) {
		const int i = threadIdx.x + k * BS;
		if (i < N) out[i] = requant_code_f(f[k], requant_factor(plan.r, plan.s));
	}
	if (threadIdx.x == 0) a.out_scale[t] = plan.out;
}

// projection funnel -> residual reconcile -> (optional) RMSNorm, all on one token's row
// (forward_sites.cpp:871-989 residual; :410-459 norm).  `out_stream` never aliases `stream`.
template <int BS, int EPT, int RS>
__global__ __launch_bounds__(BS) void k_residual_norm(sslm_launch::ResidualArgs a) {
	__shared__ uint32_t s_b[BS / 64], s_r[BS / 64], s_n[BS / 64];
	__shared__ int32_t s_ss[BS / 64];
	__shared__ int64_t land[256];  // landed branch value per branch code (code + 127)
	__shared__ int32_t s_st;
	const int t = blockIdx.x, H = a.H;
	KT(0);
	const int slot = a.tok[t].slot;
	const int sidx = a.stream_idx[t], oidx = a.out_idx[t];
	const Scale bin = a.branch_in[t];
	const int32_t* bfr = a.branch_f + (size_t)t * H;
	const int8_t* srow = a.stream + (size_t)sidx * H;
	const Scale ss = a.stream_scale[sidx];
	const int32_t status0 = a.status[slot];  // broadcast from thread 0's copy below
	int32_t bf[EPT], g[EPT], sv[EPT];
	// the stream row and gains first: issued ahead of the raw planes, they share its round trip
	load_row<BS>(srow, H, sv);
	{  // without a norm the gain loads read this token's branch row (H valid int32) and are dropped:
	   // no branch around them, so nothing waits on them here
		const int32_t* gsrc = a.gain ? a.gain : (RS > 0 ? a.raw.part + (size_t)t * a.raw.ld : bfr);
		load_row<BS>(gsrc, H, g);
		int32_t gmask = a.gain ? -1 : 0;
		asm volatile("" : "+v"(gmask));  // opaque: the loads cannot be sunk into a branch on the mask
#pragma unroll
		for (int k = 0; k < EPT; ++k) g[k] &= gmask;
	}
	uint32_t bmx = 0;
	if (RS > 0) {
		int j[EPT];
		bool live[EPT];
		int64_t v[EPT];
#pragma unroll
		for (int k = 0; k < EPT; ++k) {
			j[k] = threadIdx.x + k * BS;
			live[k] = j[k] < H;
		}
		const bool ok = raw_row<EPT, RS>(a.raw, 0, a.M, t, j, live, v);
#pragma unroll
		for (int k = 0; k < EPT; ++k) {
			bf[k] = sat_i32(v[k]);
			bmx = max(bmx, sat_abs_u32(v[k]));
		}
		if (!ok) bmx = kBad32;
	}
	if (RS == 0) load_row<BS>(bfr, H, bf);
	if (RS == 0) bmx = part_max32_fixed<BS, (EPT + 15) / 16>(a.branch_maxpart, 0, H / 16, t);
	if (threadIdx.x == 0) s_st = status0;
	bmx = blk_max32<BS>(bmx, s_b);
	KT(1);
	if (s_st != 0) return;
	FunnelPlan bplan;
	int32_t st = bmx == kBad32 ? kBiasReconcileProductOutOfDomain : funnel_plan(bmx, &bin, 1, a.branch_site, &bplan);
	if (st == kOk && !fits_i32(ss.m)) st = kCarriedScaleMantissaOutOfDomain;
	if (st != kOk) {
		if (threadIdx.x == 0) set_status(a.status, slot, a.layer, st);
		return;
	}
	KT(2);
	// The landed value depends on the branch code alone (forward_sites.cpp:513-653 with the
	// row's scales fixed), so the 255 possible values are tabulated, one per thread;
	// INT64_MIN marks a code whose landing exceeds int64.
	int32_t code[EPT];
#pragma unroll
	for (int k = 0; k < EPT; ++k) code[k] = requant_code_f(bf[k], requant_factor(bplan.r, bplan.s));
	if (a.branch_tap.codes) {
#pragma unroll
		for (int k = 0; k < EPT; ++k) {
			const int i = threadIdx.x + k * BS;
			if (i < H) a.branch_tap.codes[(size_t)t * a.branch_tap.ld + i] = (int8_t)code[k];
		}
		if (threadIdx.x == 0) a.branch_tap.scale[t] = bplan.out;
	}
	if (threadIdx.x < 255) {
		const int64_t r_h = reciprocal_fast(ss.m);
		const int64_t kx = composed_exponent(bplan.out.e, ss.e);
		bool cl, ex;
		const int64_t rec = landing_small((int64_t)threadIdx.x - 127, bplan.out.m, r_h, kx, &cl, &ex);
		land[threadIdx.x] = ex ? kI64Min : rec;
	}
	__syncthreads();
	int64_t w[EPT];
	uint32_t mx = 0;
#pragma unroll
	for (int k = 0; k < EPT; ++k) {
		const int i = threadIdx.x + k * BS;
		w[k] = 0;
		if (i < H) {
			const int64_t rec = land[code[k] + 127];
			if (rec == kI64Min) {
				mx = kBad32;
			} else {
				w[k] = rec + sv[k];
				mx = max(mx, sat_abs_u32(w[k]));
			}
		}
	}
	mx = blk_max32<BS>(mx, s_r);
	KT(3);
	FunnelPlan rplan;
	st = mx == kBad32 ? kResidualReconciliationMagnitudeOutOfDomain : funnel_plan(mx, &ss, 1, a.res_site, &rplan);
	if (st != kOk) {
		if (threadIdx.x == 0) set_status(a.status, slot, a.layer, st);
		return;
	}
	KT(4);
	int8_t* out = a.out_stream + (size_t)oidx * H;
	int32_t c[EPT];
#pragma unroll
	for (int k = 0; k < EPT; ++k) {
		const int i = threadIdx.x + k * BS;
		c[k] = 0;
		if (i < H) {
			c[k] = requant_code_f(w[k], requant_factor(rplan.r, rplan.s));
			out[i] = (int8_t)c[k];
		}
	}
	if (threadIdx.x == 0) a.out_stream_scale[oidx] = rplan.out;
	KT(5);
	if (a.gain) {
		const int32_t st2 = rmsnorm_regs<BS, EPT>(c, g, H, a.norm_site, a.norm_out + (size_t)t * H, &a.norm_scale[t],
		                                          a.norm_recip ? &a.norm_recip[t] : nullptr, s_ss, s_n, nullptr);
		if (threadIdx.x == 0 && st2 > 0) set_status(a.status, slot, a.layer, st2);
	}
	KT(6);
}

// debug taps of the gate and up funnels: columns [j0, j1) of row t, thread-strided as the callers
// hold them; `scales`: this block also writes the row's two scales
template <int BS, int EPT>
__device__ __forceinline__ void tap_gate_up_impl(const sslm_launch::ActArgs& a, int t, int j0, int j1,
                                                 const int32_t (&gc)[EPT], const int32_t (&uc)[EPT], Scale gs,
                                                 Scale us, bool scales) {
#pragma unroll
	for (int k = 0; k < EPT; ++k) {
		const int i = j0 + threadIdx.x + k * BS;
		if (i < j1) {
			a.gate_tap.codes[(size_t)t * a.gate_tap.ld + i] = (int8_t)gc[k];
			a.up_tap.codes[(size_t)t * a.up_tap.ld + i] = (int8_t)uc[k];
		}
	}
	if (scales && threadIdx.x == 0) {
		a.gate_tap.scale[t] = gs;
		a.up_tap.scale[t] = us;
	}
}

// gate/up funnels -> MlpActSite (forward_sites.cpp:796-864) -> act funnel.  The sigmoid of a
// gate code depends only on the code and the token's gate scale, so the 256 possible values
// are tabulated per block once the gate plan is known.
// Rows of up to 9 elements per thread fit in 64 VGPRs: two 1024-thread rows per CU, so a 512-row
// prefill chunk runs in one round over the CUs.
template <int BS, int EPT, int RS>
__global__ __launch_bounds__(BS) __attribute__((amdgpu_waves_per_eu(RS == 0 && EPT <= 9 ? 2048 / BS * BS / 256 : 1)))
void k_mlp_act(sslm_launch::ActArgs a) {
	__shared__ uint32_t s_gu[2 * BS / 64], s_a[BS / 64];
	__shared__ int32_t sig[256];
	__shared__ int32_t s_silu[1025];  // the SiLU node table, loaded with the row
	__shared__ int32_t s_st;
	const int t = xcd_row(blockIdx.x, gridDim.x), I = a.I;
	const int slot = a.tok[t].slot;
	const int32_t* gfr = a.gu_f + (size_t)t * 2 * I;
	const int32_t* ufr = gfr + I;
	int32_t gf[EPT], uf[EPT];
	uint32_t gm = 0, um = 0;
	// Without raw planes the plans need only the tile maxima: those, the SiLU table, the scale
	// and the status word are issued first and the rows after them, so the reductions, the
	// plans and the sigmoid table run while the rows are in flight.
	int32_t sv[(1025 + BS - 1) / BS];
#pragma unroll
	for (int k = 0; k < (1025 + BS - 1) / BS; ++k) sv[k] = a.silu[min((int)threadIdx.x + k * BS, 1024)];
	if (RS == 0) {
		gm = part_max32_fixed<BS, (EPT + 15) / 16>(a.gu_maxpart, 0, I / 16, t);
		um = part_max32_fixed<BS, (EPT + 15) / 16>(a.gu_maxpart, I / 16, I / 16, t);
	}
	const Scale inc = a.in_scale[t];
	const int32_t st0 = a.status[slot];
	int32_t gv[EPT], uv[EPT];
	if (RS == 0) {
		// every wave's small loads ahead of any wave's row loads in the CU's memory queue
		__syncthreads();
		load_row_raw<BS>(gfr, I, gv);
		load_row_raw<BS>(ufr, I, uv);
	}
	if (RS > 0) {
		int jg[EPT], ju[EPT];
		bool live[EPT];
		int64_t vg[EPT], vu[EPT];
#pragma unroll
		for (int k = 0; k < EPT; ++k) {
			jg[k] = threadIdx.x + k * BS;
			ju[k] = I + jg[k];
			live[k] = jg[k] < I;
		}
		const bool okg = raw_row<EPT, RS>(a.raw, 0, a.M, t, jg, live, vg);
		const bool oku = raw_row<EPT, RS>(a.raw, 1, a.M, t, ju, live, vu);
#pragma unroll
		for (int k = 0; k < EPT; ++k) {
			gf[k] = sat_i32(vg[k]);
			uf[k] = sat_i32(vu[k]);
			gm = max(gm, sat_abs_u32(vg[k]));
			um = max(um, sat_abs_u32(vu[k]));
		}
		if (!(okg && oku)) gm = kBad32;
	}
#pragma unroll
	for (int k = 0; k < (1025 + BS - 1) / BS; ++k)
		if (threadIdx.x + k * BS < 1025) s_silu[threadIdx.x + k * BS] = sv[k];
	if (threadIdx.x == 0) s_st = st0;
	blk_max32x2<BS>(gm, um, s_gu);
	if (s_st != 0) return;
	FunnelPlan gp, up;
	int32_t st = gm == kBad32 ? kBiasReconcileProductOutOfDomain : funnel_plan(gm, &inc, 1, a.gate_site, &gp);
	if (st == kOk) st = funnel_plan(um, &inc, 1, a.up_site, &up);
	if (st == kOk) st = check_silu_scale(gp.out.m, gp.out.e);
	if (st != kOk) {
		if (threadIdx.x == 0) set_status(a.status, slot, a.layer, st);
		return;
	}
	const Scale gs = gp.out;
	if (threadIdx.x < 256) sig[threadIdx.x] = silu_sigmoid_q15(s_silu, (int8_t)(threadIdx.x - 128), gs.m, (int)gs.e);
	if (RS == 0) {
		row_take<BS>(gv, I, gf);
		row_take<BS>(uv, I, uf);
	}
	int32_t gc[EPT], uc[EPT];
#pragma unroll
	for (int k = 0; k < EPT; ++k) {
		gc[k] = requant_code_f(gf[k], requant_factor(gp.r, gp.s));
		uc[k] = requant_code_f(uf[k], requant_factor(up.r, up.s));
	}
	if (a.gate_tap.codes) tap_gate_up_impl<BS, EPT>(a, t, 0, I, gc, uc, gp.out, up.out, true);
	__syncthreads();
	// The loader admits only the canonical SiLU table (values in [0, 32768]) and the sigmoid
	// interpolates between its entries, so |code * sig * code| <= 127 * 32768 * 127 < 2^31.
	int32_t w[EPT];
	uint32_t mx = 0;
#pragma unroll
	for (int k = 0; k < EPT; ++k) {
		w[k] = gc[k] * sig[gc[k] + 128] * uc[k];
		mx = max(mx, (uint32_t)abs(w[k]));
	}
	mx = blk_max32<BS>(mx, s_a);
	const Scale inc2[2] = {gp.out, up.out};
	FunnelPlan ap;
	st = funnel_plan(mx, inc2, 2, a.act_site, &ap);
	if (st != kOk) {
		if (threadIdx.x == 0) set_status(a.status, slot, a.layer, st);
		return;
	}
	int8_t* act = a.act + (size_t)t * I;
#pragma unroll
	for (int k = 0; k < EPT; ++k) {
		const int i = threadIdx.x + k * BS;
		if (i < I) act[i] = requant_code_f(w[k], requant_factor(ap.r, ap.s));
	}
	if (threadIdx.x == 0) a.act_scale[t] = ap.out;
}

// 16-column tiles of a gate or up row the sliced SiLU reads maxima of (I <= 20480, row_geometry_ok)
constexpr int kActSliceTiles = 20480 / 16;

// mlp_act over column slices (forward_sites.cpp:796-869): block (t, s) takes columns
// [s * per, (s + 1) * per) of row t.  Part 1: the gate and up funnels from the projection's
// tile maxima (every block derives the same plans), the SiLU-LUT sigmoid table, the products
// and the slice's maximum; the block of slice 0 keeps the gate and up scales for part 2.
template <int BS, int EPT>
__global__ __launch_bounds__(BS) void k_mlp_act_s1(sslm_launch::ActArgs a, int per) {
	__shared__ uint32_t s_gu[2 * BS / 64], s_a[BS / 64];
	__shared__ int32_t sig[256];
	__shared__ int32_t s_silu[1025];
	__shared__ int32_t s_st;
	const int t = blockIdx.x, sl = blockIdx.y, I = a.I;
	const int slot = a.tok[t].slot;
	const int j0 = sl * per, j1 = min(I, j0 + per);
	const int32_t* gfr = a.gu_f + (size_t)t * 2 * I;
	const int32_t* ufr = gfr + I;
	// The tile maxima (I / 16 <= kActSliceTiles per row), the SiLU table, the scale and the status
	// word as straight-line loads, then the slice (clamped to it): the plans need only the former,
	// so the reductions, the plans and the sigmoid table run while the slice is in flight.
	uint32_t gm = part_max32_fixed<BS, (kActSliceTiles + BS - 1) / BS>(a.gu_maxpart, 0, I / 16, t);
	uint32_t um = part_max32_fixed<BS, (kActSliceTiles + BS - 1) / BS>(a.gu_maxpart, I / 16, I / 16, t);
	const Scale inc = a.in_scale[t];
	const int32_t st0 = a.status[slot];
	int32_t sv[(1025 + BS - 1) / BS];
#pragma unroll
	for (int k = 0; k < (1025 + BS - 1) / BS; ++k) sv[k] = a.silu[min((int)threadIdx.x + k * BS, 1024)];
	int32_t gv[EPT], uv[EPT];
#pragma unroll
	for (int k = 0; k < EPT; ++k) {
		const int i = j0 + min((int)threadIdx.x + k * BS, j1 - j0 - 1);
		gv[k] = gfr[i];
		uv[k] = ufr[i];
	}
	// the status word held from here: left to the compiler, its load sinks below the slice's and
	// thread 0's store to LDS waits for the whole slice before the reduction
	asm volatile("" ::"s"(st0));
#pragma unroll
	for (int k = 0; k < (1025 + BS - 1) / BS; ++k)
		if (threadIdx.x + k * BS < 1025) s_silu[threadIdx.x + k * BS] = sv[k];
	if (threadIdx.x == 0) s_st = st0;
	blk_max32x2<BS>(gm, um, s_gu);
	if (s_st != 0) return;
	FunnelPlan gp, up;
	int32_t st = funnel_plan(gm, &inc, 1, a.gate_site, &gp);
	if (st == kOk) st = funnel_plan(um, &inc, 1, a.up_site, &up);
	if (st == kOk) st = check_silu_scale(gp.out.m, gp.out.e);
	if (st != kOk) {
		if (threadIdx.x == 0) set_status(a.status, slot, a.layer, st);
		return;
	}
	const Scale gs = gp.out;
	if (threadIdx.x < 256) sig[threadIdx.x] = silu_sigmoid_q15(s_silu, (int8_t)(threadIdx.x - 128), gs.m, (int)gs.e);
	int32_t gf[EPT], uf[EPT];
#pragma unroll
	for (int k = 0; k < EPT; ++k) {
		const bool in = j0 + (int)threadIdx.x + k * BS < j1;
		gf[k] = in ? gv[k] : 0;
		uf[k] = in ? uv[k] : 0;
	}
	int32_t gc[EPT], uc[EPT];
#pragma unroll
	for (int k = 0; k < EPT; ++k) {
		gc[k] = requant_code_f(gf[k], requant_factor(gp.r, gp.s));
		uc[k] = requant_code_f(uf[k], requant_factor(up.r, up.s));
	}
	if (a.gate_tap.codes) tap_gate_up_impl<BS, EPT>(a, t, j0, j1, gc, uc, gp.out, up.out, sl == 0);
	__syncthreads();
	uint32_t mx = 0;
	int32_t* prow = a.prod + (size_t)t * I;
#pragma unroll
	for (int k = 0; k < EPT; ++k) {
		const int i = j0 + threadIdx.x + k * BS;
		const int32_t w = gc[k] * sig[gc[k] + 128] * uc[k];  // < 2^31: canonical SiLU table, as in k_mlp_act
		if (i < j1) {
			prow[i] = w;
			mx = max(mx, (uint32_t)abs(w));
		}
	}
	mx = blk_max32<BS>(mx, s_a);
	if (threadIdx.x == 0) {
		a.act_maxpart[(size_t)sl * kPartLd + t] = mx;
		if (sl == 0) {
			a.gu_scale[2 * t] = gp.out;
			a.gu_scale[2 * t + 1] = up.out;
		}
	}
}

// Part 2: the act funnel over the slices' maxima (every block derives the same plan) and the
// slice's codes; slice 0 writes the row's act scale.
template <int BS, int EPT>
__global__ __launch_bounds__(BS) void k_mlp_act_s2(sslm_launch::ActArgs a, int per) {
	__shared__ int32_t s_st;
	const int t = blockIdx.x, sl = blockIdx.y, I = a.I, S = gridDim.y;
	const int slot = a.tok[t].slot;
	const int j0 = sl * per, j1 = min(I, j0 + per);
	const int32_t* prow = a.prod + (size_t)t * I;
	int32_t w[EPT];
#pragma unroll
	for (int k = 0; k < EPT; ++k) {
		const int i = j0 + threadIdx.x + k * BS;
		w[k] = i < j1 ? prow[i] : 0;
	}
	uint32_t mx = 0;  // over the S slices' maxima: straight-line loads from clamped indices
#pragma unroll
	for (int i = 0; i < sslm_launch::kMaxActSlices; ++i) mx = max(mx, a.act_maxpart[(size_t)min(i, S - 1) * kPartLd + t]);
	const Scale inc2[2] = {a.gu_scale[2 * t], a.gu_scale[2 * t + 1]};
	if (threadIdx.x == 0) s_st = a.status[slot];
	__syncthreads();
	if (s_st != 0) return;
	FunnelPlan ap;
	const int32_t st = funnel_plan(mx, inc2, 2, a.act_site, &ap);
	if (st != kOk) {
		if (threadIdx.x == 0) set_status(a.status, slot, a.layer, st);
		return;
	}
	int8_t* act = a.act + (size_t)t * I;
#pragma unroll
	for (int k = 0; k < EPT; ++k) {
		const int i = j0 + threadIdx.x + k * BS;
		if (i < j1) act[i] = requant_code_f(w[k], requant_factor(ap.r, ap.s));
	}
	if (threadIdx.x == 0 && sl == 0) a.act_scale[t] = ap.out;
}

// Attention for one (query head, token): the head's query against positions [0, pos]
// (forward_sites.cpp:1791-1905).  Scores, i-exp values and Q15 probabilities of the row live in
// LDS when the context fits (else in the per-launch global scratch); each thread owns the
// positions p = threadIdx.x + k * BS through the score, exp and probability passes, so those
// passes meet only at the row max and row sum.  PV: D / 16 threads cover one V row (16 channels
// each); the position groups' int32 partials meet in LDS (exact: probabilities sum to <= 2^15).
//
// FUSED (decode): the block first does the q|k|v post-processing of qkv_post for its head --
// the q funnel from the projection's tile maxima, q codes and RoPE(q), and the K/V landing and
// RoPE(K) of its KV group at the current position (forward_sites.cpp:1281-1418, :1748-1787).
// The group's first head writes that K/V to the cache; every head reads position `pos` from its
// own LDS copy, so no block reads what another block of the launch writes.
// LDSROW: the row's scores / i-exp values / probabilities live in LDS (else in the launch's global
// scratch).  A compile-time choice: one pointer that may address either space is a generic one,
// and its flat accesses count in both wait counters, so every LDS wait would also wait for the
// K/V loads in flight.
template <int BS, int D, bool FUSED, bool LDSROW>
__global__ __launch_bounds__(BS) void k_attention(sslm_launch::AttnArgs a) {
	extern __shared__ int64_t dyn[];
	__shared__ int64_t s_mx[BS / 64];
	__shared__ int64_t s_sum[BS / 64];
	__shared__ uint64_t s_ref[BS / 64];
	__shared__ uint32_t s_ab[BS / 64], s_qm[BS / 64];
	__shared__ int32_t s_ctx[BS * 16];  // pass 4 partial sums: PG position groups x D
	__shared__ __attribute__((aligned(16))) int8_t s_qc[D], s_kc[D], s_vc[D];
	__shared__ int32_t s_st;
	__shared__ int64_t s_cst[5];  // FUSED: the i-exp constants and their status (one thread derives them)
	__shared__ int32_t s_vd;      // FUSED: the q funnel's verdict
	constexpr int TPR = D / 16, PG = BS / TPR, PAIRS = D / 2;  // pass 4: threads per row, row groups
	static_assert(BS >= PAIRS, "one thread per RoPE pair");
	// XCD-aware order: workgroups go round-robin to the 8 XCDs (block id mod 8), so the R query
	// heads of one (kv head, token) group are numbered id = (i * R + r) * 8 + x -- all on XCD x,
	// sharing that XCD's L2 copy of the group's K/V.  Ids past the last group exit at once.
	const int group = a.NH / a.NKV;
	int h, t;
	{
		const int id = blockIdx.x, x = id & 7, k = id >> 3;
		const int gi = x + 8 * (k / group);  // group index: (token, kv head) = (gi / NKV, gi % NKV)
		if (gi >= a.M * a.NKV) return;
		t = gi / a.NKV;
		h = (gi % a.NKV) * group + k % group;
	}
	const int kvh = h / group;
	const TokenInfo ti = a.tok[t];
	const int64_t km = a.khead_m[kvh], ke = a.khead_e[kvh];
	const int32_t* cf = a.ctx_fold + 3 * h;
	const int32_t f0 = cf[0], f1 = cf[1], f2 = cf[2];
	const int64_t pos = ti.pos;
	const int8_t* blk = a.kv_pool + (int64_t)ti.block * a.block_bytes;
	const int64_t half = a.cap * (int64_t)a.NKV * D;
	int8_t* kstore = a.kv_pool + (int64_t)ti.block * a.block_bytes + (int64_t)a.layer * half * 2 + (int64_t)kvh * a.cap * D;
	// The K row this thread scores first (position threadIdx.x) and the V rows it multiplies first
	// (positions pg + i * PG, dimensions 16 dq .. + 15) are issued right after the loads of the
	// q|k|v post-processing: the cache rows before `pos` do not depend on it, so their round trip
	// overlaps it.  (Loads complete in order for the wait counter, so the post-processing's own
	// loads go first, unconditionally, and nothing waits on a load issued after the prefetch.)  In
	// the fused form position `pos` itself is written by this launch and is read from LDS instead,
	// so it is never loaded here (its slot loads row 0, unused).
	constexpr int VPF = 2;  // V rows per thread issued ahead
	const int8_t* kbase = blk + (int64_t)a.layer * half * 2 + (int64_t)kvh * a.cap * D;
	const int8_t* vbase = kbase + half;
	const int dq = threadIdx.x % TPR, pg = threadIdx.x / TPR;
	v4i kpre[D / 16], vpre[VPF];
	auto prefetch = [&]() {
		const int64_t width_est = pos + 1;
		const int64_t p0 = threadIdx.x;
		const int64_t pr = (p0 < width_est && (!FUSED || p0 != pos) && p0 < a.cap) ? p0 : 0;
#pragma unroll
		for (int j = 0; j < D / 16; ++j) kpre[j] = load16(kbase + pr * D + 16 * j);
#pragma unroll
		for (int i = 0; i < VPF; ++i) {
			const int64_t p = pg + (int64_t)i * PG;
			const int64_t pv = (p < width_est && (!FUSED || p != pos) && p < a.cap) ? p : 0;
			vpre[i] = load16(vbase + pv * D + 16 * dq);
		}
	};
	v4i q[D / 16];
	Scale qs;
	if (!FUSED) {
		qs = a.q_scale[t];
		const int8_t* qrow = a.q_rot + (size_t)t * a.H + (size_t)h * D;
#pragma unroll
		for (int j = 0; j < D / 16; ++j) q[j] = load16(qrow + 16 * j);
		if (threadIdx.x == 0) s_st = a.status[ti.slot];
		prefetch();
	} else {
		const int H = a.H, KVH = a.NKV * D, i = threadIdx.x;
		// the KV head's scalar constants and the status word first: their round trip overlaps the
		// vector loads below instead of following them
		const int64_t rtk = a.r_t_k[kvh], rtv = a.r_t_v[kvh], etk = a.e_t_k[kvh], etv = a.e_t_v[kvh];
		const int32_t status0 = a.status[ti.slot];
		const Scale ns = a.in_scale[t];
		const bool pos_ok = pos >= 0 && pos < a.cap;
		// The independent jobs of the post-processing run on different waves: q codes and RoPE(q)
		// on threads [0, PAIRS) (after the q funnel's plan), the K landing and RoPE(K) on the last
		// PAIRS threads and the V landing on [PAIRS, 2 PAIRS) when that range is free (else on the
		// K threads), neither waiting for the plan.  The i-exp constants need the plan and are
		// derived by one thread after the post-processing barrier, while pass 1 runs; nothing
		// reads them before pass 1's reduction.  Each thread's loads are unconditional from
		// clamped indices (see the prefetch above); pair index ic is its q, K or V pair.
		constexpr int LB = BS - PAIRS;  // first K landing thread
		constexpr bool SPLITV = 3 * PAIRS < BS;  // V landing on threads [PAIRS, 2 PAIRS)
		constexpr int CST = LB - 1 >= (SPLITV ? 2 * PAIRS : PAIRS) ? LB - 1 : BS - 1;  // i-exp constants
		const bool kthr = i >= LB, vthr = SPLITV ? (i >= PAIRS && i < 2 * PAIRS) : kthr;
		const int ntq = H / 16;
		const int ic = i < PAIRS ? i : (kthr ? i - LB : (vthr ? i - PAIRS : 0));
		const uint32_t qm0 = a.q_maxpart[(size_t)(i < ntq ? i : ntq - 1) * kPartLd + t];
		int2 qv = ((const int2*)(a.q_f + (size_t)t * H + (size_t)h * D))[ic];
		const int64_t* kvrow = a.kv_f + (size_t)t * 2 * KVH + (size_t)kvh * D;
		longlong2 kk = ((const longlong2*)kvrow)[ic], vv = ((const longlong2*)(kvrow + KVH))[ic];
		const int64_t pp = pos_ok ? pos : 0;
		int32_t c = (int32_t)a.rope_cos[pp * PAIRS + ic], sn = (int32_t)a.rope_sin[pp * PAIRS + ic];
		prefetch();
		uint32_t qmx = i < ntq ? qm0 : 0u;
		for (int k2 = i + BS; k2 < ntq; k2 += BS) qmx = max(qmx, a.q_maxpart[(size_t)k2 * kPartLd + t]);
		const int64_t k_e = composed_exponent(ns.e, etk), v_e = composed_exponent(ns.e, etv);
		// one reading of the status word for the whole block (another block may set it meanwhile)
		if (threadIdx.x == 0) s_st = status0;
		qmx = blk_max32<BS>(qmx, s_qm);
		if (s_st != 0) return;
		uint32_t sat = 0;
		char2 kc = make_char2(0, 0), vc = make_char2(0, 0);
		if (kthr) {  // the K landing and RoPE(K) of pair ic
			bool c0, c1, x0;
			const int64_t k0 = clamp_code(landing_rescale(kk.x, ns.m, rtk, k_e, &c0, &x0));
			const int64_t k1 = clamp_code(landing_rescale(kk.y, ns.m, rtk, k_e, &c1, &x0));
			int64_t xr, yr;
			rope_pair((int32_t)k0, (int32_t)k1, c, sn, &xr, &yr);
			kc = make_char2((char)clamp_code(xr), (char)clamp_code(yr));
			sat += (uint32_t)c0 + (uint32_t)c1;
			((char2*)s_kc)[ic] = kc;
		}
		if (vthr) {  // the V landing of pair ic
			bool c2, c3, x0;
			vc = make_char2((char)clamp_code(landing_rescale(vv.x, ns.m, rtv, v_e, &c2, &x0)),
			                (char)clamp_code(landing_rescale(vv.y, ns.m, rtv, v_e, &c3, &x0)));
			sat += (uint32_t)c2 + (uint32_t)c3;
			((char2*)s_vc)[ic] = vc;
		}
		// the q funnel's plan, on the waves that use it (wave-uniform condition)
		FunnelPlan plan{};
		if (i < PAIRS || (i >> 6) == (CST >> 6)) {
			int32_t st = funnel_plan(qmx, &ns, 1, a.q_site, &plan);
			if (st == kOk && !pos_ok) st = kPositionOverCap;
			if (threadIdx.x == 0) {  // the verdict, the same for every head of the token
				s_vd = st;
				if (st != kOk) set_status(a.status, ti.slot, a.layer, st);
			}
			if (st == kOk && i < PAIRS) {  // q codes and RoPE(q) of pair i
				int64_t xr, yr;
				const int32_t x = requant_code_f(qv.x, requant_factor(plan.r, plan.s));
				const int32_t y = requant_code_f(qv.y, requant_factor(plan.r, plan.s));
				rope_pair(x, y, c, sn, &xr, &yr);
				((char2*)s_qc)[i] = make_char2((char)clamp_code(xr), (char)clamp_code(yr));
			}
		}
		__syncthreads();
		if (s_vd != kOk) return;  // the plan refused: no K/V store, no saturation count
		if (h % group == 0) {  // the group's writer stores the landed K/V and counts its saturations
			const int64_t off = pos * D + 2 * ic;
			if (kthr) *(char2*)(kstore + off) = kc;
			if (vthr) *(char2*)(kstore + half + off) = vc;
			const int32_t ws = wave_sum32((int32_t)sat);
			if ((threadIdx.x & 63) == 0 && ws) atomicAdd(&a.sat[ti.slot], (unsigned long long)ws);
		}
		if ((i >> 6) == (CST >> 6)) {  // the i-exp constants of the row's scale: wave-uniform, so scalar code
			const Scale qsp = plan.out;
			int64_t q0 = 0, q1 = 0, q2 = 0, q3 = 0;
			int32_t cst = kOk;
			if (!fits_i32(qsp.m) || !fits_i32(km)) {
				cst = kCarriedScaleMantissaOutOfDomain;
			} else {
				const Scale sm = combine_scale(qsp, Scale{km, ke});
				if (!fits_i32(sm.m)) cst = kCarriedScaleMantissaOutOfDomain;
				else if (iexp_scale_constants(sm.m, sm.e, a.ln2_q, a.b_q, a.ca_q, &q0, &q1, &q2) != 0)
					cst = kIExpScaleDerivationOutOfDomain;
				else {
					cst = check_softmax_width(q1, q2, pos + 1);
					q3 = softmax_ceiling(q1, q2);
				}
			}
			if (i == CST) {
				s_cst[0] = q0;
				s_cst[1] = q1;
				s_cst[2] = q2;
				s_cst[3] = q3;
				s_cst[4] = cst;
			}
		}
#pragma unroll
		for (int j = 0; j < D / 16; ++j) q[j] = *(const v4i*)(s_qc + 16 * j);
		if (a.q_tap.codes) {
			if (threadIdx.x < D) a.q_tap.codes[(size_t)t * a.q_tap.ld + (size_t)h * D + threadIdx.x] = s_qc[threadIdx.x];
			if (threadIdx.x == 0 && h == 0) a.q_tap.scale[t] = plan.out;
		}
	}
	// i-exp constants of the row's scale (FUSED: derived by one thread during pass 1 and read
	// after its reduction; else every thread, redundantly)
	int32_t st = kOk;
	int64_t c_qln2 = 0, c_qb = 0, c_qc = 0, c_M = 0;
	const int64_t width = pos + 1;
	if (FUSED) {
	} else if (!fits_i32(qs.m) || !fits_i32(km)) {
		st = kCarriedScaleMantissaOutOfDomain;
	} else {
		const Scale sm = combine_scale(qs, Scale{km, ke});
		if (!fits_i32(sm.m)) {
			st = kCarriedScaleMantissaOutOfDomain;
		} else if (iexp_scale_constants(sm.m, sm.e, a.ln2_q, a.b_q, a.ca_q, &c_qln2, &c_qb, &c_qc) != 0) {
			st = kIExpScaleDerivationOutOfDomain;
		} else {
			st = check_softmax_width(c_qb, c_qc, width);
			c_M = softmax_ceiling(c_qb, c_qc);
		}
	}
	const bool live = (FUSED || st == kOk) && width >= 1 && width <= a.cap;
	int64_t* ex = LDSROW ? dyn : a.scratch + ((int64_t)t * a.NH + h) * a.cap;
	// pass 1: scores (int32-exact dots) and the row max; the first position's row was issued at entry
	int64_t mx = INT64_MIN;
	if (live) {
#pragma unroll 2
		for (int64_t p = threadIdx.x; p < width; p += BS) {
			const int8_t* kr = kbase + p * D;
			const bool first = p == (int64_t)threadIdx.x;
			int32_t acc = 0;
#pragma unroll
			for (int j = 0; j < D / 16; ++j) {
				const v4i kw = FUSED && p == pos ? *(const v4i*)(s_kc + 16 * j) : (first ? kpre[j] : load16(kr + 16 * j));
				acc = __builtin_amdgcn_sdot4(q[j].x, kw.x, acc, false);
				acc = __builtin_amdgcn_sdot4(q[j].y, kw.y, acc, false);
				acc = __builtin_amdgcn_sdot4(q[j].z, kw.z, acc, false);
				acc = __builtin_amdgcn_sdot4(q[j].w, kw.w, acc, false);
			}
			ex[p] = acc;
			mx = acc > mx ? acc : mx;
		}
	}
	mx = blk_max_i64<BS>(mx, s_mx);
	if (!FUSED && s_st != 0) return;
	if (FUSED) {
		c_qln2 = s_cst[0];
		c_qb = s_cst[1];
		c_qc = s_cst[2];
		c_M = s_cst[3];
		st = (int32_t)s_cst[4];
	}
	if (st != kOk) {
		if (threadIdx.x == 0) report_head(a.head_status, ti.slot, h, st);
		return;
	}
	if (!live) {  // width outside [1, cap]: the KV landing of this position already refused it
		if (threadIdx.x == 0) report_head(a.head_status, ti.slot, h, kPositionOverCap);
		return;
	}
	// pass 2: i-exp values (SoftmaxRowQ15, intmath.cpp:853-889) and the row sum
	int64_t sum = 0;
	uint64_t refused = 0;
	const double inv_ln2 = c_qln2 >= 1 ? 1.0 / (double)c_qln2 : 0.0;
	// the row passed check_softmax_width; the 32-bit form where its constants allow
	if (iexp_small_ok(c_qln2, c_qb, c_M)) {
		for (int64_t p = threadIdx.x; p < width; p += BS) {
			int64_t v = iexp_small(ex[p] - mx, (int32_t)c_qln2, inv_ln2, (int32_t)c_qb, c_qc, c_M);
			refused |= v < 0 ? 1u : 0u;
			v = v < 0 ? 0 : v;
			ex[p] = v;
			sum += v;
		}
	} else {
		for (int64_t p = threadIdx.x; p < width; p += BS) {
			int64_t v = iexp_fast(ex[p] - mx, c_qln2, inv_ln2, c_qb, c_qc, c_M);
			refused |= v < 0 ? 1u : 0u;
			v = v < 0 ? 0 : v;
			ex[p] = v;
			sum += v;
		}
	}
	sum = wave_sum_i64(sum);
	refused = wave_max_u64(refused);
	if ((threadIdx.x & 63) == 0) {
		s_sum[threadIdx.x >> 6] = sum;
		s_ref[threadIdx.x >> 6] = refused;
	}
	__syncthreads();
	sum = 0;
	refused = 0;
#pragma unroll
	for (int i = 0; i < BS / 64; ++i) {
		sum += s_sum[i];
		refused |= s_ref[i];
	}
	if (refused) {
		if (threadIdx.x == 0) report_head(a.head_status, ti.slot, h, kSoftmaxKernelRefusedAfterGateAccepted);
		return;
	}
	// pass 3: Q15 probabilities p = (e << 15) / max(total, 1)
	const int64_t denom = sum > 1 ? sum : 1;
	const double dinv = 1.0 / (double)denom;  // e <= total: quotients at most 2^15
	if (div_q15_small_ok(denom)) {
		const double dd = (double)denom;
		for (int64_t p = threadIdx.x; p < width; p += BS) ex[p] = ex[p] == 0 ? 0 : div_q15_small(ex[p], dd, dinv);
	} else {
		for (int64_t p = threadIdx.x; p < width; p += BS) ex[p] = ex[p] == 0 ? 0 : div_rcp(ex[p] << 15, denom, dinv, 32768);
	}
	__syncthreads();
	// pass 4: context = sum_p prob * V[p].  A thread owns 16 dimensions (one 16-byte load per
	// row) of every PG-th position; the loop is unrolled so several rows are in flight.  The sums
	// are exact in int32: the probabilities of a row add up to at most 2^15.
	int32_t acc[16];
#pragma unroll
	for (int j = 0; j < 16; ++j) acc[j] = 0;
	{
		const int8_t* vc = vbase + 16 * dq;
		// the first VPF rows of this thread were issued at entry
#pragma unroll
		for (int i = 0; i < VPF; ++i) {
			const int64_t p = pg + (int64_t)i * PG;
			if (p < width) {
				const v4i v = FUSED && p == pos ? *(const v4i*)(s_vc + 16 * dq) : vpre[i];
				const int32_t pr = (int32_t)ex[p];
#pragma unroll
				for (int w = 0; w < 4; ++w) {
					const int32_t x = v[w];
					acc[4 * w] += pr * (int32_t)(int8_t)(x & 0xff);
					acc[4 * w + 1] += pr * (int32_t)(int8_t)((x >> 8) & 0xff);
					acc[4 * w + 2] += pr * (int32_t)(int8_t)((x >> 16) & 0xff);
					acc[4 * w + 3] += pr * (x >> 24);
				}
			}
		}
#pragma unroll 4
		for (int64_t p = pg + (int64_t)VPF * PG; p < width; p += PG) {
			const v4i v = FUSED && p == pos ? *(const v4i*)(s_vc + 16 * dq) : load16(vc + p * D);
			const int32_t pr = (int32_t)ex[p];
#pragma unroll
			for (int w = 0; w < 4; ++w) {
				const int32_t x = v[w];
				acc[4 * w] += pr * (int32_t)(int8_t)(x & 0xff);
				acc[4 * w + 1] += pr * (int32_t)(int8_t)((x >> 8) & 0xff);
				acc[4 * w + 2] += pr * (int32_t)(int8_t)((x >> 16) & 0xff);
				acc[4 * w + 3] += pr * (x >> 24);
			}
		}
		int32_t* sc = s_ctx + pg * D + 16 * dq;
#pragma unroll
		for (int j = 0; j < 16; ++j) sc[j] = acc[j];
	}
	__syncthreads();
	uint32_t mabs = 0;
	if (threadIdx.x < D) {
		int32_t c = 0;
#pragma unroll 8
		for (int g2 = 0; g2 < PG; ++g2) c += s_ctx[g2 * D + threadIdx.x];
		const int64_t f = apply_fold(c, f0, f1, f2);
		a.ctx_f[(size_t)t * a.H + (size_t)h * D + threadIdx.x] = sat_i32(f);
		mabs = sat_abs_u32(f);
	}
	mabs = blk_max32<BS>(mabs, s_ab);
	if (threadIdx.x == 0) a.ctx_maxpart[(size_t)h * kPartLd + t] = mabs;
}

// Prefill attention over query tiles: one block per (query head, 16 consecutive tokens of one
// sequence), the same arithmetic as k_attention (forward_sites.cpp:1791-1905) with each K and V
// row read once per tile instead of once per token.  Scores Q.K^T are int32-exact on
// v_mfma_i32_16x16x64_i8 (A = the tile's 16 query rows, B = 16 key rows; any k order shared by
// both operands gives the same integer sum).  The softmax stays exact without keeping the row:
// pass 1 takes each token's row max, pass 2 recomputes the scores for the i-exp values and their
// sum, pass 3 recomputes them once more for the Q15 probabilities and multiplies by V.  P.V runs
// on the same MFMA: a probability (0 .. 2^15) is split into three 7-bit parts p = a*2^14 + b*2^7
// + c, each an int8 operand, and the three int32 products recombine exactly (the true sum is
// below 2^22 in magnitude).  V rows are staged in LDS as stored ([position][dim]) and read with
// gfx950's byte-transposing LDS load, so a lane's 16 B operand holds 16 positions of one dimension.
// The launch must hold one sequence's consecutive positions (a prefill chunk).
constexpr int kTiledECache = 512;  // positions whose i-exp values an 8-wave tiled-attention block keeps

template <int D, int NW>
__global__ __launch_bounds__(64 * NW, NW == 4 ? 3 : 1) void k_attention_tiled(sslm_launch::AttnArgs a) {
	constexpr int TQ = 16, KB = 16 * NW, NC = (D + 63) / 64, DT = D / 16, PS = KB + 16, VS = D + 16;
	__shared__ __attribute__((aligned(16))) int8_t s_p[3][TQ][PS];  // probability parts [part][token][pos]
	__shared__ __attribute__((aligned(16))) int8_t s_v[KB][VS];     // the current step's V rows, padded
	__shared__ int64_t s_c[TQ][4];                                   // per token: q_ln2, q_b, q_c, ceiling
	__shared__ double s_inv[TQ];                                     // per token: 1 / q_ln2
	__shared__ int64_t s_red[NW][TQ];
	__shared__ int32_t s_pos[TQ], s_ok[TQ];
	__shared__ uint32_t s_mab[TQ], s_rf[TQ];  // per token: |context| maximum, softmax refused
	__shared__ int32_t s_st;
	// 8-wave blocks keep pass 2's i-exp values for rows up to kTiledECache positions, so pass 3
	// neither recomputes the scores nor the i-exp values; each lane reads back only what it wrote
	constexpr int ECP = NW == 8 ? kTiledECache : 1;
	__shared__ int64_t s_e[NW == 8 ? TQ : 1][ECP];
	const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, ri = lane & 15, g = lane >> 4;
	const int group = a.NH / a.NKV, ntiles = (a.M + TQ - 1) / TQ;
	int h, tile;
	{  // XCD-aware order as in k_attention: the R heads of one (tile, kv head) share an XCD
		const int id = blockIdx.x, x = id & 7, k = id >> 3;
		const int gi = x + 8 * (k / group);
		if (gi >= ntiles * a.NKV) return;
		tile = ntiles - 1 - gi / a.NKV;  // the longest causal rows start first
		h = (gi % a.NKV) * group + k % group;
	}
	const int t0 = tile * TQ, nt = min(TQ, a.M - t0);
	const int kvh = h / group;
	const TokenInfo ti0 = a.tok[t0];
	if (threadIdx.x == 0) s_st = a.status[ti0.slot];
	if (threadIdx.x < TQ) {
		// the token's i-exp constants and width, as k_attention derives them
		const int tq = threadIdx.x;
		int32_t st = kOk;
		int64_t c0 = 0, c1 = 0, c2 = 0, cm = 0, pos = -1;
		if (tq < nt) {
			const Scale qs = a.q_scale[t0 + tq];
			pos = a.tok[t0 + tq].pos;
			const int64_t km = a.khead_m[kvh], ke = a.khead_e[kvh];
			if (!fits_i32(qs.m) || !fits_i32(km)) {
				st = kCarriedScaleMantissaOutOfDomain;
			} else {
				const Scale sm = combine_scale(qs, Scale{km, ke});
				if (!fits_i32(sm.m)) st = kCarriedScaleMantissaOutOfDomain;
				else if (iexp_scale_constants(sm.m, sm.e, a.ln2_q, a.b_q, a.ca_q, &c0, &c1, &c2) != 0)
					st = kIExpScaleDerivationOutOfDomain;
				else {
					st = check_softmax_width(c1, c2, pos + 1);
					cm = softmax_ceiling(c1, c2);
				}
			}
			if (st == kOk && !(pos + 1 >= 1 && pos + 1 <= a.cap)) st = -1;
		} else {
			st = -2;  // past the launch's last token
		}
		s_c[tq][0] = c0;
		s_c[tq][1] = c1;
		s_c[tq][2] = c2;
		s_c[tq][3] = cm;
		s_inv[tq] = st == kOk && c0 >= 1 ? 1.0 / (double)c0 : 0.0;
		s_pos[tq] = (int32_t)pos;
		s_ok[tq] = st;
		s_mab[tq] = 0;
		s_rf[tq] = 0;
	}
	__syncthreads();
	if (s_st != 0) return;
	if (threadIdx.x < nt && s_ok[threadIdx.x] != kOk)
		report_head(a.head_status, ti0.slot, h, s_ok[threadIdx.x] == -1 ? kPositionOverCap : s_ok[threadIdx.x]);
	int wmax = 0;  // positions [0, wmax) cover every live token's row
	for (int tq = 0; tq < nt; ++tq)
		if (s_ok[tq] == kOk) wmax = max(wmax, s_pos[tq] + 1);
	if (wmax == 0) return;
	const int8_t* kbase = a.kv_pool + (int64_t)ti0.block * a.block_bytes + (int64_t)a.layer * a.cap * a.NKV * D * 2 +
	                      (int64_t)kvh * a.cap * D;
	const int8_t* vbase = kbase + a.cap * (int64_t)a.NKV * D;
	// this lane's A operand: query row ri, bytes c*64 + g*16 of chunk c
	v4i qa[NC];
#pragma unroll
	for (int c = 0; c < NC; ++c) {
		const int off = c * 64 + g * 16;
		qa[c] = ri < nt && off < D ? load16(a.q_rot + (size_t)(t0 + ri) * a.H + (size_t)h * D + off) : v4i{0, 0, 0, 0};
	}
	// the output tokens of this lane: g*4 + v
	int32_t tpos[4];
	bool tok_ok[4];
#pragma unroll
	for (int v = 0; v < 4; ++v) {
		tpos[v] = s_pos[g * 4 + v];
		tok_ok[v] = s_ok[g * 4 + v] == kOk;
	}
	const int nblk = (wmax + KB - 1) / KB;
	const bool ecache = NW == 8 && nblk * KB <= ECP;
	auto scores = [&](int blk, int* p_out) {
		const int p = blk * KB + wave * 16 + ri;
		const int8_t* kr = kbase + (int64_t)min(p, (int)a.cap - 1) * D;
		v4i acc = v4i{0, 0, 0, 0};
#pragma unroll
		for (int c = 0; c < NC; ++c) {
			const int off = c * 64 + g * 16;
			const v4i kb = off < D ? load16(kr + off) : v4i{0, 0, 0, 0};
			acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(qa[c], kb, acc, 0, 0, 0);
		}
		*p_out = p;
		return acc;
	};
	// pass 1: row maxima
	int32_t mx[4] = {INT32_MIN, INT32_MIN, INT32_MIN, INT32_MIN};
	for (int blk = 0; blk < nblk; ++blk) {
		int p;
		const v4i s = scores(blk, &p);
#pragma unroll
		for (int v = 0; v < 4; ++v)
			if (tok_ok[v] && p <= tpos[v]) mx[v] = max(mx[v], s[v]);
	}
#pragma unroll
	for (int v = 0; v < 4; ++v) {
		for (int o = 8; o > 0; o >>= 1) mx[v] = max(mx[v], __shfl_xor(mx[v], o, 16));
		if (ri == 0) s_red[wave][g * 4 + v] = mx[v];
	}
	__syncthreads();
	int64_t rmx[4];
#pragma unroll
	for (int v = 0; v < 4; ++v) {
		const int tq = g * 4 + v;
		rmx[v] = s_red[0][tq];
#pragma unroll
		for (int w = 1; w < NW; ++w) rmx[v] = max(rmx[v], s_red[w][tq]);
	}
	int64_t cq[4][4];
	double inv[4];
	bool esmall[4];  // the token's constants admit iexp_small
#pragma unroll
	for (int v = 0; v < 4; ++v) {
#pragma unroll
		for (int i = 0; i < 4; ++i) cq[v][i] = s_c[g * 4 + v][i];
		inv[v] = s_inv[g * 4 + v];
		esmall[v] = iexp_small_ok(cq[v][0], cq[v][1], cq[v][3]);
	}
	auto iexp_tok = [&](int v, int64_t shifted) {
		return esmall[v] ? iexp_small(shifted, (int32_t)cq[v][0], inv[v], (int32_t)cq[v][1], cq[v][2], cq[v][3])
		                 : iexp_fast(shifted, cq[v][0], inv[v], cq[v][1], cq[v][2], cq[v][3]);
	};
	__syncthreads();
	// pass 2: i-exp values (SoftmaxRowQ15, intmath.cpp:853-889) and the row sums
	int64_t sum[4] = {0, 0, 0, 0};
	uint32_t refused = 0;
	for (int blk = 0; blk < nblk; ++blk) {
		int p;
		const v4i s = scores(blk, &p);
#pragma unroll
		for (int v = 0; v < 4; ++v) {
			if (tok_ok[v] && p <= tpos[v]) {
				const int64_t e = iexp_tok(v, (int64_t)s[v] - rmx[v]);
				if (ecache) s_e[NW == 8 ? g * 4 + v : 0][NW == 8 ? p : 0] = e;
				if (e < 0) refused |= 1u << v;
				else sum[v] += e;
			}
		}
	}
#pragma unroll
	for (int v = 0; v < 4; ++v) {
		for (int o = 8; o > 0; o >>= 1) sum[v] += __shfl_xor(sum[v], o, 16);
		if (ri == 0) s_red[wave][g * 4 + v] = sum[v];
	}
	for (int o = 8; o > 0; o >>= 1) refused |= __shfl_xor(refused, o, 16);
	if (ri == 0 && refused)
		for (int v = 0; v < 4; ++v)
			if (refused >> v & 1) s_rf[g * 4 + v] = 1;
	__syncthreads();
	int64_t denom[4];
	double dinv[4], ddn[4];
	bool dsmall[4];  // the token's total admits div_q15_small
#pragma unroll
	for (int v = 0; v < 4; ++v) {
		const int tq = g * 4 + v;
		int64_t tot = 0;
#pragma unroll
		for (int w = 0; w < NW; ++w) tot += s_red[w][tq];
		denom[v] = tot > 1 ? tot : 1;
		dinv[v] = 1.0 / (double)denom[v];
		dsmall[v] = div_q15_small_ok(denom[v]);
		ddn[v] = (double)denom[v];
		tok_ok[v] = tok_ok[v] && s_rf[tq] == 0;
	}
	if (threadIdx.x < nt && s_ok[threadIdx.x] == kOk && s_rf[threadIdx.x] != 0)
		report_head(a.head_status, ti0.slot, h, kSoftmaxKernelRefusedAfterGateAccepted);
	// pass 3: Q15 probabilities p = (e << 15) / max(total, 1), then context += P . V
	constexpr int DTW = (DT + NW - 1) / NW;  // dimension tiles per wave
	v4i cacc[DTW][3];
#pragma unroll
	for (int i = 0; i < DTW; ++i)
#pragma unroll
		for (int k = 0; k < 3; ++k) cacc[i][k] = v4i{0, 0, 0, 0};
	// a step's V rows are issued before its probabilities are computed and stored to LDS after
	// them (16-byte copies; rows past the cap repeat the last one)
	constexpr int VCH = KB * (D / 16), VPT = (VCH + 64 * NW - 1) / (64 * NW);  // V chunks per thread
	for (int blk = 0; blk < nblk; ++blk) {
		v4i vr[VPT];
#pragma unroll
		for (int u = 0; u < VPT; ++u) {
			const int c = min((int)threadIdx.x + u * 64 * NW, VCH - 1);
			const int64_t pos = min(blk * KB + c / (D / 16), (int)a.cap - 1);
			vr[u] = load16(vbase + pos * D + (c % (D / 16)) * 16);
		}
		int p;
		v4i s = v4i{0, 0, 0, 0};
		if (ecache) p = blk * KB + wave * 16 + ri;
		else s = scores(blk, &p);
		const int pl = wave * 16 + ri;
#pragma unroll
		for (int v = 0; v < 4; ++v) {
			int32_t pr = 0;
			if (tok_ok[v] && p <= tpos[v]) {
				// e <= total, so the quotient is at most 2^15
				const int64_t e = ecache ? s_e[NW == 8 ? g * 4 + v : 0][NW == 8 ? p : 0] : iexp_tok(v, (int64_t)s[v] - rmx[v]);
				pr = e == 0 ? 0
				            : (dsmall[v] ? div_q15_small(e, ddn[v], dinv[v]) : (int32_t)div_rcp(e << 15, denom[v], dinv[v], 32768));
			}
			s_p[0][g * 4 + v][pl] = (int8_t)(pr >> 14);
			s_p[1][g * 4 + v][pl] = (int8_t)((pr >> 7) & 127);
			s_p[2][g * 4 + v][pl] = (int8_t)(pr & 127);
		}
		// the step's V rows, as stored
#pragma unroll
		for (int u = 0; u < VPT; ++u) {
			const int c = (int)threadIdx.x + u * 64 * NW;
			if (c < VCH) *(v4i*)&s_v[c / (D / 16)][(c % (D / 16)) * 16] = vr[u];
		}
		__syncthreads();
#pragma unroll
		for (int i = 0; i < DTW; ++i) {
			const int dt = wave + NW * i;
			if (dt < DT) {
#pragma unroll
				for (int kk = 0; kk < KB / 64; ++kk) {
					// B operand (dimension dt*16 + ri, positions kk*64 + 16g + 0..15) by two LDS
					// transpose reads: in each 16-lane group, lane m names the 8 bytes at row
					// (position) m/2, dimensions dt*16 + 8(m%2) + 0..7, and lane ri receives byte
					// ri%8 of rows 2j + ri/8, j = 0..7 -- dimension dt*16 + ri at 8 positions
					const int8_t* vp = &s_v[kk * 64 + g * 16 + (ri >> 1)][dt * 16 + 8 * (ri & 1)];
					const v2i lo = __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) v2i*)vp);
					const v2i hi =
					    __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) v2i*)(vp + 8 * VS));
					const v4i b = v4i{lo.x, lo.y, hi.x, hi.y};
#pragma unroll
					for (int k = 0; k < 3; ++k) {
						const v4i pa = *(const v4i*)&s_p[k][ri][kk * 64 + g * 16];
						cacc[i][k] = __builtin_amdgcn_mfma_i32_16x16x64_i8(pa, b, cacc[i][k], 0, 0, 0);
					}
				}
			}
		}
		__syncthreads();
	}
	// epilogue: recombine the parts, fold, store; the per-token maximum over the head's dims
	const int32_t* cf = a.ctx_fold + 3 * h;
	const int32_t f0 = cf[0], f1 = cf[1], f2 = cf[2];
#pragma unroll
	for (int i = 0; i < DTW; ++i) {
		const int dt = wave + NW * i;
		if (dt < DT) {
			const int d = dt * 16 + ri;
#pragma unroll
			for (int v = 0; v < 4; ++v) {
				const int32_t c = (int32_t)(((uint32_t)cacc[i][0][v] << 14) + ((uint32_t)cacc[i][1][v] << 7) +
				                            (uint32_t)cacc[i][2][v]);
				const int64_t f = apply_fold(c, f0, f1, f2);
				const int tq = g * 4 + v;
				if (tok_ok[v]) a.ctx_f[(size_t)(t0 + tq) * a.H + (size_t)h * D + d] = sat_i32(f);
				const uint32_t m = dpp_max16(tok_ok[v] ? sat_abs_u32(f) : 0u);
				if (ri == 0 && tok_ok[v]) atomicMax(&s_mab[tq], m);
			}
		}
	}
	__syncthreads();
	if (threadIdx.x < nt && s_ok[threadIdx.x] == kOk && s_rf[threadIdx.x] == 0)
		a.ctx_maxpart[(size_t)h * kPartLd + t0 + threadIdx.x] = s_mab[threadIdx.x];
}

// Decode attention over long contexts, one block per (token, KV head): the KV group's G query
// heads are the rows of the MFMA tiles, so each K and V row is read once for all of them.  One
// block per (query head, token) reads every K/V byte G times (7 at the 7B shape); at ~2,000
// positions those re-reads, served by L2 and the memory-side cache, were what bounded the
// per-head kernel.  The arithmetic is k_attention's (forward_sites.cpp:1791-1905), element by
// element:
//   * prologue: the q|k|v post-processing of the fused kernel for the whole group -- the q funnel
//     from the projection's tile maxima, q codes and RoPE(q) of the G heads, and the K/V landing
//     and RoPE(K) of the KV head at `pos`, which this block alone writes to the cache and keeps in
//     LDS (no block reads what another writes);
//   * pass 1: int32-exact scores Q.K^T on v_mfma_i32_16x16x64_i8 (A = the G query rows, zero rows
//     past G; B = 16 key rows), kept in LDS ([G][cap] int32) with the row maxima; K rows are
//     issued a group of steps ahead of the group being scored;
//   * pass 2: i-exp values and row sums over every (row, position), spread over all threads; then
//     the Q15 probabilities, each overwriting its score as three 7-bit parts;
//   * pass 3: per step of KB positions, the parts staged as int8 MFMA operands, V rows staged in
//     LDS as stored (issued a group of steps ahead) and P.V on MFMA through gfx950's
//     byte-transposing LDS read, as k_attention_tiled does;
//   * epilogue: per head the ctx fold, outputs and the per-head tile maximum.
// Refusals are reported per head exactly as the per-head kernel reports them.
template <int D, int NW, int GM>
__global__ __launch_bounds__(64 * NW, 1) void k_attention_group(sslm_launch::AttnArgs a) {
	constexpr int TQ = 16, BS = 64 * NW, KB = 16 * NW, NC = (D + 63) / 64, DT = D / 16, PS = KB + 16, VS = D + 16;
	constexpr int PAIRS = D / 2, DTW = (DT + NW - 1) / NW, VCH = KB * (D / 16), VPT = (VCH + BS - 1) / BS;
	// K and V rows are issued R steps at a time, one group of R steps ahead of the one consumed:
	// a step's rows alone (16 KB per block at D = 128) leave the CU waiting a round trip per step
	constexpr int R = D <= 128 ? 4 : 2, RK = R;  // V and K steps per group
	extern __shared__ __attribute__((aligned(16))) int32_t s_sc[];     // [G][wcap] scores
	__shared__ __attribute__((aligned(16))) int8_t s_p[2][3][TQ][PS];  // probability parts [buffer][part][row][pos]
	__shared__ __attribute__((aligned(16))) int8_t s_v[2][KB][VS];     // V rows [buffer][pos][dim]
	__shared__ __attribute__((aligned(16))) int8_t s_qc[TQ][D];     // the rows' rotated q codes
	__shared__ __attribute__((aligned(16))) int8_t s_kc[D], s_vc[D];
	__shared__ int64_t s_red[NW][TQ];
	__shared__ uint32_t s_qm[NW], s_mab[TQ], s_rf[TQ];
	__shared__ int32_t s_st, s_rmx[TQ];
	__shared__ int32_t s_dump[BS];  // where rows G .. GM - 1 of the softmax loops store
	__shared__ int64_t s_cst[5];     // the rows' i-exp constants and their status (one thread derives them)
	__shared__ int32_t s_vd;         // the q plan's verdict
	const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, ri = lane & 15, g = lane >> 4, i = threadIdx.x;
	const int H = a.H, KVH = a.NKV * D, GG = a.NH / a.NKV;
	// a.row_halves = 2: two blocks per (token, KV group), numbered 16 k + 8 h + x (x < 8) for group
	// 8 k + x and row half h, so both halves sit on XCD x (blocks go to the XCDs round-robin) and
	// the second reads the group's K/V from that XCD's L2; ids past the last group exit
	int gi = blockIdx.x, rh = 0;
	if (a.row_halves == 2) {
		gi = (blockIdx.x >> 4) * 8 + (blockIdx.x & 7);
		rh = (blockIdx.x >> 3) & 1;
		if (gi >= a.M * a.NKV) return;
	}
	const int t = gi / a.NKV, kvh = gi % a.NKV;
	// this block's rows: heads h0 .. h0 + G - 1 of the group (all of them, or one half)
	const int gh = a.row_halves == 2 ? (GG + 1) / 2 : GG;
	const int G = rh == 0 ? gh : GG - gh, h0 = kvh * GG + rh * gh;
	const TokenInfo ti = a.tok[t];
	// the KV head's scalar constants and the status word first: their round trip overlaps the
	// vector loads below instead of following them
	const int64_t rtk = a.r_t_k[kvh], rtv = a.r_t_v[kvh], etk = a.e_t_k[kvh], etv = a.e_t_v[kvh];
	const int64_t km = a.khead_m[kvh], ke = a.khead_e[kvh];
	const int32_t status0 = a.status[ti.slot];
	const int64_t pos = ti.pos, width = pos + 1, cap = a.cap;
	const bool pos_ok = pos >= 0 && pos < cap;
	const int64_t half = cap * (int64_t)KVH;
	const int8_t* kbase = a.kv_pool + (int64_t)ti.block * a.block_bytes + (int64_t)a.layer * half * 2 + (int64_t)kvh * cap * D;
	const int8_t* vbase = kbase + half;
	// ---- prologue loads, unconditional from clamped indices, then the first K step ahead ----
	const int ntq = H / 16;
	const uint32_t qm0 = a.q_maxpart[(size_t)(i < ntq ? i : ntq - 1) * kPartLd + t];
	const int qi = i < G * PAIRS ? i : G * PAIRS - 1, qr = qi / PAIRS, qj = qi % PAIRS;
	const int2 qv = ((const int2*)(a.q_f + (size_t)t * H + (size_t)(h0 + qr) * D))[qj];
	// The prologue's independent jobs run on different waves: q codes on threads [0, G PAIRS)
	// after the q plan, the K landing and RoPE(K) on the last PAIRS threads and the V landing on
	// the PAIRS threads before them when the q codes leave those free (else on the K threads),
	// neither waiting for the plan.  The i-exp constants, which only pass 2 needs, are derived by
	// thread 0 at the start of pass 1 and read after pass 1's reduction.
	constexpr int LB = BS - PAIRS;  // first K landing thread
	const bool kthr = i >= LB;
	const bool splitv = G * PAIRS <= LB - PAIRS;  // block-uniform
	const bool vthr = splitv ? (i >= LB - PAIRS && i < LB) : kthr;
	const int ki = kthr ? i - LB : (vthr ? i - (LB - PAIRS) : 0);
	const int64_t* kvrow = a.kv_f + (size_t)t * 2 * KVH + (size_t)kvh * D;
	const longlong2 kk = ((const longlong2*)kvrow)[ki], vv = ((const longlong2*)(kvrow + KVH))[ki];
	const int64_t pp = pos_ok ? pos : 0;
	const int32_t cq = (int32_t)a.rope_cos[pp * PAIRS + qj], sq = (int32_t)a.rope_sin[pp * PAIRS + qj];
	const int32_t ck = (int32_t)a.rope_cos[pp * PAIRS + ki], sk = (int32_t)a.rope_sin[pp * PAIRS + ki];
	const Scale ns = a.in_scale[t];
	// the ctx fold parameters of this lane's output rows (heads h0 + 4 g + v), for the epilogue
	int32_t f0[4], f1[4], f2[4];
#pragma unroll
	for (int v = 0; v < 4; ++v) {
		const int r = g * 4 + v;
		const int32_t* cf = a.ctx_fold + 3 * (h0 + (r < G ? r : 0));
		f0[v] = cf[0];
		f1[v] = cf[1];
		f2[v] = cf[2];
	}
	auto load_k = [&](int blk, v4i (&kb)[NC]) {
		const int64_t p = (int64_t)blk * KB + wave * 16 + ri;
		const int64_t pr = p < width && p != pos && p < cap ? p : 0;
#pragma unroll
		for (int c = 0; c < NC; ++c) {
			const int off = c * 64 + g * 16;
			kb[c] = off < D ? load16(kbase + pr * D + off) : v4i{0, 0, 0, 0};
		}
	};
	v4i kb0[RK][NC], kb1[RK][NC];
	auto load_kr = [&](int c0, v4i (&kb)[RK][NC]) {
#pragma unroll
		for (int j = 0; j < RK; ++j) load_k(c0 * RK + j, kb[j]);
	};
	load_kr(0, kb0);
	uint32_t qmx = i < ntq ? qm0 : 0u;
	for (int k2 = i + BS; k2 < ntq; k2 += BS) qmx = max(qmx, a.q_maxpart[(size_t)k2 * kPartLd + t]);
	const int64_t k_e = composed_exponent(ns.e, etk), v_e = composed_exponent(ns.e, etv);
	// one reading of the status word for the whole block (another block of the token may set it
	// while this one runs)
	if (i == 0) s_st = status0;
	for (int k2 = i; k2 < TQ * D / 16; k2 += BS) ((v4i*)&s_qc[0][0])[k2] = v4i{0, 0, 0, 0};
	for (int k2 = i; k2 < 2 * 3 * TQ * PS / 16; k2 += BS) ((v4i*)&s_p[0][0][0][0])[k2] = v4i{0, 0, 0, 0};
	if (i < TQ) {
		s_mab[i] = 0;
		s_rf[i] = 0;
	}
	qmx = blk_max32<BS>(qmx, s_qm);
	if (s_st != 0) return;
	// K/V landing of this KV head at pos: every block of the group keeps it in LDS; row half 0's
	// writes it to the cache and counts its saturations once the plan has passed (no block reads
	// what another writes)
	uint32_t sat = 0;
	char2 kc = make_char2(0, 0), vc = make_char2(0, 0);
	if (kthr) {
		bool c0, c1, x0;
		const int64_t k0 = clamp_code(landing_rescale(kk.x, ns.m, rtk, k_e, &c0, &x0));
		const int64_t k1 = clamp_code(landing_rescale(kk.y, ns.m, rtk, k_e, &c1, &x0));
		int64_t xr, yr;
		rope_pair((int32_t)k0, (int32_t)k1, ck, sk, &xr, &yr);
		kc = make_char2((char)clamp_code(xr), (char)clamp_code(yr));
		sat += (uint32_t)c0 + (uint32_t)c1;
		((char2*)s_kc)[ki] = kc;
	}
	if (vthr) {
		bool c2, c3, x0;
		vc = make_char2((char)clamp_code(landing_rescale(vv.x, ns.m, rtv, v_e, &c2, &x0)),
		                (char)clamp_code(landing_rescale(vv.y, ns.m, rtv, v_e, &c3, &x0)));
		sat += (uint32_t)c2 + (uint32_t)c3;
		((char2*)s_vc)[ki] = vc;
	}
	// the q plan on the q threads (whole waves when G PAIRS is a multiple of 64)
	FunnelPlan plan{};
	if (i < G * PAIRS) {
		int32_t st0 = funnel_plan(qmx, &ns, 1, a.q_site, &plan);
		if (st0 == kOk && !pos_ok) st0 = kPositionOverCap;
		if (i == 0) {  // the verdict, the same for every head of the token
			s_vd = st0;
			if (st0 != kOk) set_status(a.status, ti.slot, a.layer, st0);
		}
		if (st0 == kOk) {  // q codes and RoPE of the group's heads
			int64_t xr, yr;
			const int32_t x = requant_code_f(qv.x, requant_factor(plan.r, plan.s));
			const int32_t y = requant_code_f(qv.y, requant_factor(plan.r, plan.s));
			rope_pair(x, y, cq, sq, &xr, &yr);
			*(char2*)&s_qc[qr][2 * qj] = make_char2((char)clamp_code(xr), (char)clamp_code(yr));
		}
	}
	__syncthreads();
	if (s_vd != kOk) return;
	if (rh == 0) {  // the group's writer
		int8_t* kstore = const_cast<int8_t*>(kbase);
		const int64_t off = pos * D + 2 * ki;
		if (kthr) *(char2*)(kstore + off) = kc;
		if (vthr) *(char2*)(kstore + half + off) = vc;
		const int32_t ws = wave_sum32((int32_t)sat);
		if (lane == 0 && ws) atomicAdd(&a.sat[ti.slot], (unsigned long long)ws);
	}
	const Scale qs = plan.out;
	// i-exp constants of the rows' common scale (the q scale is the token's, km / ke the KV
	// head's), read after pass 1's reduction
	if (i == 0) {
		int64_t q0 = 0, q1 = 0, q2 = 0, q3 = 0;
		int32_t cst = kOk;
		if (!fits_i32(qs.m) || !fits_i32(km)) {
			cst = kCarriedScaleMantissaOutOfDomain;
		} else {
			const Scale sm = combine_scale(qs, Scale{km, ke});
			if (!fits_i32(sm.m)) cst = kCarriedScaleMantissaOutOfDomain;
			else if (iexp_scale_constants(sm.m, sm.e, a.ln2_q, a.b_q, a.ca_q, &q0, &q1, &q2) != 0)
				cst = kIExpScaleDerivationOutOfDomain;
			else {
				cst = check_softmax_width(q1, q2, width);
				q3 = softmax_ceiling(q1, q2);
			}
		}
		s_cst[0] = q0;
		s_cst[1] = q1;
		s_cst[2] = q2;
		s_cst[3] = q3;
		s_cst[4] = cst;
	}
	if (a.q_tap.codes) {
		for (int k2 = i; k2 < G * D; k2 += BS) a.q_tap.codes[(size_t)t * a.q_tap.ld + (size_t)h0 * D + k2] = s_qc[k2 / D][k2 % D];
		if (i == 0 && kvh == 0 && rh == 0) a.q_tap.scale[t] = qs;
	}
	// (width <= wcap holds by construction: the host sizes wcap from the launch's positions; the
	// passed plan implies width <= cap)
	if (!(width >= 1 && width <= cap && width <= a.wcap)) {
		if (i < G) report_head(a.head_status, ti.slot, h0 + i, kPositionOverCap);
		return;
	}
	v4i qa[NC];
#pragma unroll
	for (int c = 0; c < NC; ++c) {
		const int off = c * 64 + g * 16;
		qa[c] = off < D ? *(const v4i*)&s_qc[ri][off] : v4i{0, 0, 0, 0};
	}
	// ---- pass 1: scores and row maxima ----
	const int nblk = (int)((width + KB - 1) / KB);
	const int64_t cstride = a.wcap;  // a multiple of KB, at least every width of the launch
	int32_t mx[4] = {INT32_MIN, INT32_MIN, INT32_MIN, INT32_MIN};
	auto score_step = [&](int blk, v4i (&kb)[NC]) {
		const int64_t p = (int64_t)blk * KB + wave * 16 + ri;
		v4i acc = v4i{0, 0, 0, 0};
#pragma unroll
		for (int c = 0; c < NC; ++c) {
			const int off = c * 64 + g * 16;
			const v4i b = p == pos && off < D ? *(const v4i*)(s_kc + off) : kb[c];
			acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(qa[c], b, acc, 0, 0, 0);
		}
		if (p < width) {
#pragma unroll
			for (int v = 0; v < 4; ++v) {
				const int r = g * 4 + v;
				if (r < G) {
					s_sc[(int64_t)r * cstride + p] = acc[v];
					mx[v] = max(mx[v], acc[v]);
				}
			}
		}
	};
	const int ngr = (nblk + RK - 1) / RK;  // groups of RK steps (steps past the row score nothing)
	auto score_group = [&](int c0, v4i (&kb)[RK][NC]) {
#pragma unroll
		for (int j = 0; j < RK; ++j) score_step(c0 * RK + j, kb[j]);
	};
	// the group loads are unconditional (rows past the width read row 0, a cache hit): a load
	// issued on one path only would make every later wait drain all loads in flight
	for (int c0 = 0; c0 < ngr; c0 += 2) {
		load_kr(c0 + 1, kb1);
		score_group(c0, kb0);
		if (c0 + 1 >= ngr) break;
		load_kr(c0 + 2, kb0);
		score_group(c0 + 1, kb1);
	}
	// the first V steps do not depend on the softmax: they are in flight through passes 2 and 3's
	// arithmetic
	auto load_v = [&](int blk, v4i (&vr)[VPT]) {
#pragma unroll
		for (int u = 0; u < VPT; ++u) {
			const int c = i + u * BS;
			const int pr = c / (D / 16), ch = c % (D / 16);
			const int64_t p = (int64_t)blk * KB + pr;
			const int64_t pl = p < width && p != pos && p < cap ? p : 0;
			vr[u] = c < VCH ? load16(vbase + pl * D + ch * 16) : v4i{0, 0, 0, 0};
		}
	};
	v4i vr0[R][VPT], vr1[R][VPT];
	auto load_vr = [&](int c0, v4i (&vr)[R][VPT]) {
#pragma unroll
		for (int j = 0; j < R; ++j) load_v(c0 * R + j, vr[j]);
	};
	load_vr(0, vr0);
#pragma unroll
	for (int v = 0; v < 4; ++v) {
		for (int o = 8; o > 0; o >>= 1) mx[v] = max(mx[v], __shfl_xor(mx[v], o, 16));
		if (ri == 0) s_red[wave][g * 4 + v] = mx[v];
	}
	__syncthreads();
	if (i < TQ) {
		int64_t m = s_red[0][i];
		for (int w = 1; w < NW; ++w) m = max(m, s_red[w][i]);
		s_rmx[i] = (int32_t)m;
	}
	__syncthreads();
	const int64_t c_qln2 = s_cst[0], c_qb = s_cst[1], c_qc = s_cst[2], c_M = s_cst[3];
	const int32_t st = (int32_t)s_cst[4];
	if (st != kOk) {  // every head of the group: the same refusal the per-head kernel reports
		if (i < G) report_head(a.head_status, ti.slot, h0 + i, st);
		return;
	}
	// ---- pass 2: i-exp values and row sums over every (row, position) ----
	// Every row of the block has the same constants (one token's q scale, one KV head's K scale).
	// Each score's slot then keeps what the probabilities need: the i-exp value when the ceiling
	// fits 31 bits, else (32-bit constants) the packed quotient and remainder it is finished from,
	// else nothing (the value is recomputed from the score).  Positions outer, GM rows inner as
	// straight-line code: rows G .. GM - 1 repeat row G - 1's inputs, store to a per-thread dummy
	// slot and are masked out of the refusal bits (their sums are never read), so a thread's rows
	// are independent chains.
	const bool esmall = iexp_small_ok(c_qln2, c_qb, c_M), ekeep = c_M < ((int64_t)1 << 31);
	const double inv_ln2 = c_qln2 >= 1 ? 1.0 / (double)c_qln2 : 0.0;
	int32_t rmx[GM], ro[GM];  // row r's maximum and offset in s_sc (row G - 1's for padding rows)
#pragma unroll
	for (int r = 0; r < GM; ++r) {
		const int rr = r < G ? r : G - 1;
		rmx[r] = s_rmx[rr];
		ro[r] = rr * (int32_t)cstride;
	}
	// where row r stores position p: its own slot, or the dummy slot for a padding row
	auto slot = [&](int r, int64_t p) -> int32_t* { return r < G ? s_sc + ro[r] + (int32_t)p : s_dump + i; };
	const uint32_t gmask = (1u << G) - 1u;
	{
		int64_t sum[GM];
		uint32_t refused = 0;
#pragma unroll
		for (int r = 0; r < GM; ++r) sum[r] = 0;
		auto pass2 = [&](auto small) {
			for (int64_t p = i; p < width; p += BS) {
#pragma unroll
				for (int r = 0; r < GM; ++r) {
					const int64_t sh = (int64_t)s_sc[ro[r] + (int32_t)p] - rmx[r];
					int64_t e;
					int32_t keep;
					if constexpr (decltype(small)::value) {
						const uint32_t zr = iexp_small_zr(sh, (int32_t)c_qln2, inv_ln2);
						e = iexp_small_value(zr, (int32_t)c_qb, c_qc, c_M);
						keep = ekeep ? (int32_t)(e < 0 ? 0 : e) : (int32_t)zr;
					} else {
						e = iexp_fast(sh, c_qln2, inv_ln2, c_qb, c_qc, c_M);
						keep = (int32_t)(e < 0 ? 0 : e);
					}
					refused |= (e < 0 ? 1u : 0u) << r;
					sum[r] += e < 0 ? 0 : e;
					if (decltype(small)::value || ekeep) *slot(r, p) = keep;
				}
			}
		};
		if (esmall) pass2(std::true_type{});
		else pass2(std::false_type{});
		refused &= gmask;
#pragma unroll
		for (int r = 0; r < GM; ++r) {
			if (r < G) {
				const int64_t ws = wave_sum_i64(sum[r]);
				if (lane == 0) s_red[wave][r] = ws;
			}
		}
		if (refused) atomicOr(&s_rf[0], refused);  // bit r: row r refused somewhere
	}
	__syncthreads();
	const uint32_t rf = s_rf[0];
	if (i < G && (rf >> i & 1)) report_head(a.head_status, ti.slot, h0 + i, kSoftmaxKernelRefusedAfterGateAccepted);
	// Q15 probabilities p = (e << 15) / max(total, 1) of every (row, position), each overwriting
	// its slot as the three 7-bit parts p >> 14 | (p >> 7 & 127) << 8 | (p & 127) << 16 (zero for
	// a refused row).  e <= total, so a quotient is at most 2^15.
	{
		int64_t dn[GM];
		double di[GM], dd[GM];
		bool dsm = true, live_r[GM];
#pragma unroll
		for (int r = 0; r < GM; ++r) {
			const int rr = r < G ? r : G - 1;
			int64_t tot = 0;
			for (int w = 0; w < NW; ++w) tot += s_red[w][rr];
			dn[r] = tot > 1 ? tot : 1;
			di[r] = 1.0 / (double)dn[r];
			dd[r] = (double)dn[r];
			dsm = dsm && div_q15_small_ok(dn[r]);
			live_r[r] = !(rf >> rr & 1);
		}
		// kept: 0 the value, 1 the packed quotient and remainder, 2 nothing (the score)
		auto probs = [&](auto kept, auto qsmall) {
			constexpr int K = decltype(kept)::value;
			for (int64_t p = i; p < width; p += BS) {
				int32_t w[GM];
#pragma unroll
				for (int r = 0; r < GM; ++r) {
					const int32_t v = s_sc[ro[r] + (int32_t)p];
					int64_t e;
					if constexpr (K == 0) e = v;
					else if constexpr (K == 1) e = iexp_small_value((uint32_t)v, (int32_t)c_qb, c_qc, c_M);
					else e = iexp_fast((int64_t)v - rmx[r], c_qln2, inv_ln2, c_qb, c_qc, c_M);
					int32_t pr;
					if constexpr (decltype(qsmall)::value) pr = div_q15_small(e, dd[r], di[r]);
					else pr = (int32_t)div_rcp(e << 15, dn[r], di[r], 32768);
					pr = live_r[r] && e > 0 ? pr : 0;
					w[r] = (pr >> 14) | ((pr >> 7) & 127) << 8 | (pr & 127) << 16;
				}
				// every row read before any is overwritten (a padding row reads row G - 1)
#pragma unroll
				for (int r = 0; r < GM; ++r) *slot(r, p) = w[r];
			}
		};
		using I0 = std::integral_constant<int, 0>;
		using I1 = std::integral_constant<int, 1>;
		using I2 = std::integral_constant<int, 2>;
		if (ekeep && dsm) probs(I0{}, std::true_type{});
		else if (ekeep) probs(I0{}, std::false_type{});
		else if (esmall && dsm) probs(I1{}, std::true_type{});
		else if (esmall) probs(I1{}, std::false_type{});
		else probs(I2{}, std::false_type{});
	}
	__syncthreads();
	// ---- pass 3: Q15 probabilities and P.V on MFMA ----
	v4i cacc[DTW][3];
#pragma unroll
	for (int d2 = 0; d2 < DTW; ++d2)
#pragma unroll
		for (int k = 0; k < 3; ++k) cacc[d2][k] = v4i{0, 0, 0, 0};
	// Step j's operands are staged into buffer j & 1 while step j - 1's are multiplied from the
	// other one, so a step costs one barrier: buffer b was last read by the multiply before the
	// previous barrier.
	auto stage = [&](int blk, const v4i (&vr)[VPT], int b) {
		// the step's probability parts of every live row (zero past the width), four positions
		// of one row per thread: one 16-byte read of the packed parts, three 4-byte writes
#pragma unroll
		for (int u = 0; u < (TQ * KB / 4 + BS - 1) / BS; ++u) {
			const int e4 = i + u * BS;
			if (e4 < G * (KB / 4)) {
				const int r = e4 / (KB / 4), pl = 4 * (e4 % (KB / 4));
				const int64_t p = (int64_t)blk * KB + pl;
				v4i w = *(const v4i*)&s_sc[(int64_t)r * cstride + p];  // in bounds: cstride is a multiple of KB
#pragma unroll
				for (int q = 0; q < 4; ++q) w[q] = p + q < width ? w[q] : 0;
				// byte q of part k = byte k of word q
				*(int32_t*)&s_p[b][0][r][pl] = (w[0] & 0xff) | (w[1] & 0xff) << 8 | (w[2] & 0xff) << 16 | (w[3] & 0xff) << 24;
				*(int32_t*)&s_p[b][1][r][pl] = (w[0] >> 8 & 0xff) | (w[1] >> 8 & 0xff) << 8 | (w[2] >> 8 & 0xff) << 16 |
				                               (w[3] >> 8 & 0xff) << 24;
				*(int32_t*)&s_p[b][2][r][pl] = (w[0] >> 16 & 0xff) | (w[1] >> 16 & 0xff) << 8 | (w[2] >> 16 & 0xff) << 16 |
				                               (w[3] >> 16 & 0xff) << 24;
			}
		}
#pragma unroll
		for (int u = 0; u < VPT; ++u) {
			const int c = i + u * BS;
			if (c < VCH) {
				const int pr = c / (D / 16), ch = c % (D / 16);
				const int64_t p = (int64_t)blk * KB + pr;
				*(v4i*)&s_v[b][pr][ch * 16] = p == pos ? *(const v4i*)(s_vc + ch * 16) : vr[u];
			}
		}
	};
	auto multiply = [&](int b) {
#pragma unroll
		for (int d2 = 0; d2 < DTW; ++d2) {
			const int dt = wave + NW * d2;
			if (dt < DT) {
#pragma unroll
				for (int kk2 = 0; kk2 < KB / 64; ++kk2) {
					const int8_t* vp = &s_v[b][kk2 * 64 + g * 16 + (ri >> 1)][dt * 16 + 8 * (ri & 1)];
					const v2i lo = __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) v2i*)vp);
					const v2i hi =
					    __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) v2i*)(vp + 8 * VS));
					const v4i bv = v4i{lo.x, lo.y, hi.x, hi.y};
#pragma unroll
					for (int k = 0; k < 3; ++k) {
						const v4i pa = *(const v4i*)&s_p[b][k][ri][kk2 * 64 + g * 16];
						cacc[d2][k] = __builtin_amdgcn_mfma_i32_16x16x64_i8(pa, bv, cacc[d2][k], 0, 0, 0);
					}
				}
			}
		}
	};
	// V rows in groups of R steps, one group ahead: an iteration multiplies steps c0 R .. c0 R +
	// 2R - 1 (groups c0 in vr0 and c0 + 1 in vr1) and stages each next step; group c0 + 1 is issued
	// at its start (vr1's last reader was the previous iteration), group c0 + 2 once vr0's last
	// step is staged
	stage(0, vr0[0], 0);
	__syncthreads();
	// (the group loads are unconditional, as in pass 1)
	for (int c0 = 0; c0 * R < nblk; c0 += 2) {
		load_vr(c0 + 1, vr1);
#pragma unroll
		for (int jj = 0; jj < 2 * R; ++jj) {
			const int j = c0 * R + jj;
			if (jj == R - 1) load_vr(c0 + 2, vr0);
			if (j >= nblk) break;
			if (j + 1 < nblk) {
				if (jj + 1 < R) stage(j + 1, vr0[jj + 1 < R ? jj + 1 : 0], (j + 1) & 1);
				else if (jj + 1 < 2 * R) stage(j + 1, vr1[jj + 1 - R < R ? jj + 1 - R : 0], (j + 1) & 1);
				else stage(j + 1, vr0[0], (j + 1) & 1);
			}
			multiply(j & 1);
			__syncthreads();
		}
	}
	// ---- epilogue: recombine, per-head fold, store, per-head maximum ----
	bool rok[4];
#pragma unroll
	for (int v = 0; v < 4; ++v) rok[v] = g * 4 + v < G && !(rf >> (g * 4 + v) & 1);
#pragma unroll
	for (int d2 = 0; d2 < DTW; ++d2) {
		const int dt = wave + NW * d2;
		if (dt < DT) {
			const int d = dt * 16 + ri;
#pragma unroll
			for (int v = 0; v < 4; ++v) {
				const int r = g * 4 + v;
				const int32_t c = (int32_t)(((uint32_t)cacc[d2][0][v] << 14) + ((uint32_t)cacc[d2][1][v] << 7) +
				                            (uint32_t)cacc[d2][2][v]);
				const int64_t f = apply_fold(c, f0[v], f1[v], f2[v]);
				if (rok[v]) a.ctx_f[(size_t)t * H + (size_t)(h0 + r) * D + d] = sat_i32(f);
				const uint32_t m = dpp_max16(rok[v] ? sat_abs_u32(f) : 0u);
				if (ri == 0 && rok[v]) atomicMax(&s_mab[r], m);
			}
		}
	}
	__syncthreads();
	if (i < G && !(rf >> i & 1)) a.ctx_maxpart[(size_t)(h0 + i) * kPartLd + t] = s_mab[i];
}

// Bench reference: a plain streaming read of `bytes` (a multiple of 16), four 16-byte loads per
// thread in flight, XOR-reduced into a sink that is written only on an impossible value.  The
// decode GEMV bench runs it over the same weight buffers in the same launch order as the GEMV
// pass, as the HBM rate a launch sequence of that shape can reach at all.
__global__ __launch_bounds__(256) void k_stream_read(const v4i* p, int64_t nvec, int* sink) {
	int64_t i = (int64_t)blockIdx.x * 1024 + threadIdx.x;
	const int64_t stride = (int64_t)gridDim.x * 1024;
	v4i acc = v4i{0, 0, 0, 0};
	for (; i < nvec; i += stride) {
		v4i t[4];
#pragma unroll
		for (int u = 0; u < 4; ++u) t[u] = i + u * 256 < nvec ? p[i + u * 256] : v4i{0, 0, 0, 0};
#pragma unroll
		for (int u = 0; u < 4; ++u) acc ^= t[u];
	}
	if ((acc[0] ^ acc[1] ^ acc[2] ^ acc[3]) == 0x5eed5eed) sink[0] = 1;
}

// Debug capture (sslm_hip_debug_capture): row t of a site buffer, and its scale, into the
// capture area.  One block per row.
__global__ __launch_bounds__(256) void k_debug_gather(const int8_t* src, const Scale* ssrc, const int32_t* idx, int n,
                                                      int8_t* dst, Scale* sdst, int ld) {
	const int t = blockIdx.x, r = idx ? idx[t] : t;
	for (int i = threadIdx.x; i < n; i += 256) dst[(size_t)t * ld + i] = src[(size_t)r * n + i];
	if (threadIdx.x == 0) sdst[t] = ssrc[r];
}

// LoRA intermediate (forward_sites.cpp:1066-1086): u[k] = clamp(amp_fold(A[k] . x))
__global__ __launch_bounds__(kBlock) void k_lora_u(sslm_launch::LoraUArgs a) {
	// one block per (token, adapted projection); wave w computes ranks w, w + 4, ...: each lane
	// covers 16-byte chunks of K with sdot4 (|A.x| <= 127^2 * K < 2^31, exact in int32), the
	// wave reduces with DPP, lane 0 applies the u fold (UFS1) and clamps to +-127
	const int t = blockIdx.x, p = blockIdx.y;
	const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
	const int chunks = a.K >> 4;  // K is a multiple of 64
	const int8_t* x = a.x + (size_t)t * a.K;
	constexpr int kMaxChunks = 20480 / 16 / 64;  // K <= 20480: at most 20 chunks per lane
	v4i xc[kMaxChunks];
#pragma unroll
	for (int i = 0; i < kMaxChunks; ++i) {
		const int c = lane + 64 * i;
		xc[i] = c < chunks ? load16(x + 16 * c) : v4i{0, 0, 0, 0};
	}
	for (int r = wave; r < a.rank; r += kBlock / 64) {
		const int8_t* arow = a.a[p] + (size_t)r * a.K;
		int32_t acc = 0;
#pragma unroll
		for (int i = 0; i < kMaxChunks; ++i) {
			const int c = lane + 64 * i;
			if (64 * i < chunks) {  // wave-uniform bound
				const v4i w = c < chunks ? load16(arow + 16 * c) : v4i{0, 0, 0, 0};
				acc = __builtin_amdgcn_sdot4(w.x, xc[i].x, acc, false);
				acc = __builtin_amdgcn_sdot4(w.y, xc[i].y, acc, false);
				acc = __builtin_amdgcn_sdot4(w.z, xc[i].z, acc, false);
				acc = __builtin_amdgcn_sdot4(w.w, xc[i].w, acc, false);
			}
		}
		acc = wave_sum32(acc);
		if (lane == 0) {
			const int32_t* f = a.ufold[p] + 3 * r;
			a.u[p][(size_t)t * kMaxRank + r] = (int8_t)clamp_code(apply_amp_fold((int64_t)acc, f[0], f[1], f[2]));
		}
	}
}

// lowest-index argmax (forward_sites.cpp:2427-2437) from per-tile keys: the key orders by
// logit, then by the complement of the index, so the maximum key is the lowest maximal index.
// One block per token over its contiguous key row; loads go out in batches of 8 per thread.
// Damped greedy's top-k set (src/damped_greedy_topk.cpp's FsdTopK order) by radix selection:
// each element's 64-bit key -- biased logit (INT32_MIN when masked) in the high word, then the
// legal bit, then 2^31 - 1 - index -- is unique and orders like the reference's comparator, so
// the k largest keys are the candidate set.  Eight passes fix the k-th largest key a byte at a
// time from the top (a 256-bin histogram of the elements still matching the fixed prefix); a
// last pass writes every element whose key is at least that one.
constexpr int kTopKBlock = 1024;
__device__ __forceinline__ uint64_t topk_key(const int32_t* row, const uint8_t* page, int i) {
	const bool legal = !page || ((page[i >> 3] >> (i & 7)) & 1u);
	const int32_t v = legal ? row[i] : INT32_MIN;
	return ((uint64_t)((uint32_t)v ^ 0x80000000u) << 32) | ((uint64_t)legal << 31) | (uint32_t)(0x7fffffff - i);
}

__global__ __launch_bounds__(kTopKBlock) void k_topk(const int32_t* logits, int V, const uint8_t* const* mask_page,
                                                    int k, int2* out) {
	__shared__ uint32_t hist[256];
	__shared__ uint64_t s_prefix;
	__shared__ int s_need, s_count;
	const int r = blockIdx.x;
	const int32_t* row = logits + (size_t)r * V;
	const uint8_t* page = mask_page ? mask_page[r] : nullptr;
	uint64_t prefix = 0, fixed = 0;  // the k-th largest key's bits fixed so far, and their mask
	int need = k;                    // its rank among the elements matching the prefix
	for (int shift = 56; shift >= 0; shift -= 8) {
		for (int b = threadIdx.x; b < 256; b += kTopKBlock) hist[b] = 0;
		__syncthreads();
		for (int i = threadIdx.x; i < V; i += kTopKBlock) {
			const uint64_t key = topk_key(row, page, i);
			if ((key & fixed) == prefix) atomicAdd(&hist[(key >> shift) & 0xff], 1u);
		}
		__syncthreads();
		if (threadIdx.x == 0) {
			int acc = 0, b = 255;
			for (; b > 0; --b) {
				if (acc + (int)hist[b] >= need) break;
				acc += (int)hist[b];
			}
			s_need = need - acc;
			s_prefix = prefix | ((uint64_t)b << shift);
		}
		__syncthreads();
		need = s_need;
		prefix = s_prefix;
		fixed |= (uint64_t)0xff << shift;
		__syncthreads();
	}
	if (threadIdx.x == 0) s_count = 0;
	__syncthreads();
	int2* o = out + (size_t)r * k;
	for (int i = threadIdx.x; i < V; i += kTopKBlock) {
		const uint64_t key = topk_key(row, page, i);
		if (key >= prefix) {
			const int at = atomicAdd(&s_count, 1);
			if (at < k) o[at] = make_int2(i, (int32_t)((uint32_t)(key >> 32) ^ 0x80000000u));
		}
	}
}

__global__ __launch_bounds__(kRowBlock) void k_argmax_finalize(const unsigned long long* keys, int ntiles,
                                                               int32_t* out) {
	__shared__ uint64_t red[kRowBlock / 64];
	const int t = blockIdx.x;
	const unsigned long long* row = keys + (size_t)t * ntiles;
	uint64_t k = 0;
	for (int base = 0; base < ntiles; base += 8 * kRowBlock) {
		uint64_t v[8];
#pragma unroll
		for (int i = 0; i < 8; ++i) {
			const int idx = base + i * kRowBlock + (int)threadIdx.x;
			v[i] = row[min(idx, ntiles - 1)];
		}
#pragma unroll
		for (int i = 0; i < 8; ++i) k = v[i] > k ? v[i] : k;
	}
	k = blk_max<kRowBlock>(k, red);
	if (threadIdx.x == 0) out[t] = (int32_t)(0xffffffffu - (uint32_t)(k & 0xffffffffull));
}

}  // namespace sslm

// ------------------------------------------------------------------------------------------
// launch wrappers
// ------------------------------------------------------------------------------------------
namespace sslm_launch {

template <int MB, int TPW>
static void launch_gemv(const GemmArgs& g, const GemvPlan& p, hipStream_t s) {
	const dim3 grid((g.N + 16 * TPW - 1) / (16 * TPW), p.splits), block(64 * kGemvWaves);
	switch (p.cpw) {
		case 1: hipLaunchKernelGGL((k_gemv<MB, TPW, 1>), grid, block, 0, s, g, p.cps); break;
		case 2: hipLaunchKernelGGL((k_gemv<MB, TPW, 2>), grid, block, 0, s, g, p.cps); break;
		default: hipLaunchKernelGGL((k_gemv<MB, TPW, 3>), grid, block, 0, s, g, p.cps); break;
	}
}

bool gemv_eligible(int M, int K) { return M >= 1 && M <= 64 && K % 128 == 0; }

GemvPlan gemv_plan(int M, int N, int K, bool split_ok, bool raw_or_argmax) {
	GemvPlan p{};
	const int C = K / 128;
	const int tiles = (N + 15) / 16;
	if (M <= 16 && raw_or_argmax && (split_ok || tiles >= 1024)) {
		// wave-per-tile kernel: about 1024 waves (4 per CU), K split over at most
		// kMaxRawSplits planes when the consumer adds them; 3 chunks per load batch over a
		// whole-K range, up to 9 when a split's range fits one batch
		const int s = split_ok ? std::max(1, std::min({(1024 + tiles - 1) / tiles, C, kMaxRawSplits})) : 1;
		const int cps = (C + s - 1) / s;
		if (cps * 16 * 128 <= 64 * 1024) {  // the staged activations fit the default LDS limit
			p.wave_tile = true;
			p.tpw = 4;
			p.cps = cps;
			p.splits = (C + cps - 1) / cps;
			// one load batch covers a split's whole range where an instance fits it (no clamped
			// duplicate loads), else batches of 3
			p.cpw = cps <= 2 ? 2 : (cps <= 3 ? 3 : (cps <= 6 ? 6 : (cps <= 9 ? 9 : 3)));
			return p;
		}
	}
	const int mblocks = (M + 15) / 16;
	// two tiles per block halve the activation rows each block reads per weight byte; at two row
	// groups the activations are twice the weights per tile, so wide launches take it there too
	p.tpw = (mblocks <= 2 && tiles >= 1024) ? 2 : 1;
	const int blocks = (tiles + p.tpw - 1) / p.tpw;
	p.splits = 1;
	if (split_ok && blocks < kGemvTargetBlocks)
		p.splits = std::max(1, std::min({(kGemvTargetBlocks + blocks - 1) / blocks, C / kGemvWaves, kMaxRawSplits}));
	p.cps = (C + p.splits - 1) / p.splits;
	p.splits = (C + p.cps - 1) / p.cps;
	const int cpw_max = mblocks <= 2 ? 3 : 2;
	p.cpw = std::min(cpw_max, (p.cps + kGemvWaves - 1) / kGemvWaves);
	if (p.cpw < 1) p.cpw = 1;
	return p;
}

// The persistent decode GEMV takes projection launches at M <= 32 and K <= 4096 whose segments
// are funnel or wide outputs without bias or LoRA, K split nowhere (k_gemv_p).
static bool gemv_persistent_ok(const GemmArgs& g) {
	if (g.M > 32 || g.K > 4096 || g.K % 128 || g.splits > 1 || g.epi.raw_out || g.epi.argmax_key) return false;
	if (g.epi.nseg < 1 || g.epi.nseg > kMaxSeg) return false;
	for (int i = 0; i < g.epi.nseg; ++i) {
		const Segment& sg = g.epi.seg[i];
		if (sg.bias || sg.lora_b || (sg.mode != kSegFunnel && sg.mode != kSegWide)) return false;
		if (sg.n_begin % 16 || (sg.n_end % 16 && i + 1 < g.epi.nseg)) return false;
	}
	return true;
}

static int device_cus();

template <int MB>
void launch_gemv_p(const GemmArgs& g, hipStream_t s) {
	const int C = g.K >> 7, T = (g.N + 15) / 16;
	const dim3 grid(std::min(T, device_cus())), block(256);
	switch ((C + kGemvWaves - 1) / kGemvWaves) {
		case 1: hipLaunchKernelGGL((k_gemv_p<MB, 1>), grid, block, 0, s, g); break;
		case 2: hipLaunchKernelGGL((k_gemv_p<MB, 2>), grid, block, 0, s, g); break;
		case 3: hipLaunchKernelGGL((k_gemv_p<MB, 3>), grid, block, 0, s, g); break;
		case 4: hipLaunchKernelGGL((k_gemv_p<MB, 4>), grid, block, 0, s, g); break;
		case 5: hipLaunchKernelGGL((k_gemv_p<MB, 5>), grid, block, 0, s, g); break;
		case 6: hipLaunchKernelGGL((k_gemv_p<MB, 6>), grid, block, 0, s, g); break;
		case 7: hipLaunchKernelGGL((k_gemv_p<MB, 7>), grid, block, 0, s, g); break;
		default: hipLaunchKernelGGL((k_gemv_p<MB, 8>), grid, block, 0, s, g); break;
	}
}

// compute units of the current device (one persistent block each)
static int device_cus() {
	static const int n = [] {
		int dev = 0, cus = 0;
		if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
			cus = 256;
		return cus;
	}();
	return n;
}

// Every GEMM launch writes where its caller provided: raw int32 output, split-K planes, argmax
// keys, or epilogue segments with output and fold buffers that cover the columns.  Anything else
// is a caller bug that the kernels would turn into stores through null pointers: refuse it.
static void check_gemm_outputs(const GemmArgs& g) {
	bool ok = g.epi.raw_out || g.epi.argmax_key || (g.splits > 1 && g.split_part);
	if (!ok && g.epi.nseg >= 1 && g.epi.nseg <= kMaxSeg) {
		ok = g.epi.seg[0].n_begin == 0 && g.epi.seg[g.epi.nseg - 1].n_end >= g.N;
		for (int i = 0; i < g.epi.nseg; ++i) ok = ok && g.epi.seg[i].out && g.epi.seg[i].fold;
	}
	if (!ok) {
		fprintf(stderr, "sslm_hip: GEMM launch (%d x %d x %d) without a complete output\n", g.M, g.N, g.K);
		throw LaunchRefused{"gemm: incomplete output"};
	}
}

// ---- packed decode GEMVs ----
size_t packed_bytes(int N, int K) { return (size_t)((N + 15) / 16) * 16 * (size_t)K; }

void pack_gemv(const int8_t* w, int N, int K, int8_t* wp, hipStream_t s) {
	const int64_t units = (int64_t)((N + 15) / 16) * (K / 128) * 2;
	hipLaunchKernelGGL(k_pack_gemv, dim3((unsigned)((units + 3) / 4)), dim3(256), 0, s, w, N, K, wp, units);
}

constexpr int kPkMaxM = 32;  // two 16-token row groups
constexpr int kSkWaves = 8;

// tiles per block of k_gemv_pk: the smallest instance >= an even share over the CUs
static int pk_nt(int T) {
	const int need = (T + device_cus() - 1) / device_cus();
	for (int nt : {1, 2, 3, 5, 10})
		if (nt >= need) return nt;
	return 0;
}

// k_gemv_pk takes a launch without split planes or argmax keys at M <= 32, K <= 4096
static bool pk_ok(const GemmArgs& g) {
	return g.wp && g.M >= 1 && g.M <= kPkMaxM && g.K % 128 == 0 && g.K <= 4096 && !g.epi.argmax_key &&
	       g.splits <= 1 && pk_nt((g.N + 15) / 16) > 0;
}

struct SkPlan {
	int ntb, cpw, cps, splits, bx;
};

// k_gemv_sk: 8 waves of cpw chunks per split (at most kMaxRawSplits planes), ntb tiles per block
// so that about one block per CU covers the matrix
static SkPlan sk_plan(int N, int K) {
	SkPlan p{};
	const int C = K / 128, T = (N + 15) / 16;
	p.cpw = (C + kSkWaves * kMaxRawSplits - 1) / (kSkWaves * kMaxRawSplits);
	if (p.cpw > 4) return SkPlan{};
	p.cps = kSkWaves * p.cpw;
	p.splits = (C + p.cps - 1) / p.cps;
	p.ntb = std::min(8, std::max(1, (T * p.splits + device_cus() - 1) / device_cus()));
	if (p.ntb == 5) p.ntb = 6;  // instances: 1, 2, 3, 4, 6, 7, 8
	p.bx = (T + p.ntb - 1) / p.ntb;
	return p;
}

static bool sk_ok(int M, int K, const GemmArgs* g) {
	return M >= 1 && M <= kPkMaxM && K % 128 == 0 && K > 4096 && (!g || g->wp) && sk_plan(1, K).cpw > 0;
}

int gemv_raw_splits(const GemmArgs& g) {
	if (g.wp && g.M <= kPkMaxM && !g.epi.argmax_key && gemv_eligible(g.M, g.K)) {
		if (g.K <= 4096 && pk_nt((g.N + 15) / 16) > 0) return 1;
		if (sk_ok(g.M, g.K, &g)) return sk_plan(g.N, g.K).splits;
	}
	return gemv_plan(g.M, g.N, g.K, true, true).splits;
}

// chunks per wave of the k_gemv_pk instances: the smallest >= ceil(C / 4) (a larger one loads the
// last chunk again, an L2 hit, and multiplies it by zero activations)
static int pk_cpw(int C) {
	const int need = (C + kGemvWaves - 1) / kGemvWaves;
	for (int w : {1, 2, 3, 4, 7, 8})
		if (w >= need) return w;
	return 0;
}

// the epilogue form of a k_gemv_pk launch
static int pk_epi(const GemmArgs& g) {
	if (g.epi.raw_out) return kPkRaw;
	for (int i = 0; i < g.epi.nseg; ++i) {
		const Segment& sg = g.epi.seg[i];
		if (sg.mode != kSegFunnel || sg.bias || sg.lora_b || !sg.maxpart) return kPkGeneral;
	}
	return kPkFunnel;
}

template <int MB, int NT, int EPI>
static bool launch_pk_nt(const GemmArgs& g, int grid, int cpw, hipStream_t s) {
	if constexpr (MB == 2 && NT >= 5) {
		// two row groups over more than 16 chunks and several tiles per block: eight waves of 4
		// (7B gate|up at M = 32: 30.5 -> 29.1 us; with 2-3 tiles per block, q|k|v and o, the
		// larger block's fixed costs lost more: 8.6 -> 9.6 and 6.8 -> 7.5 us)
		if (cpw > 4) {
			if ((g.K / 128 + 7) / 8 > 4) return false;
			hipLaunchKernelGGL((k_gemv_pk<MB, NT, 4, EPI, 2 * kGemvWaves>), dim3(grid), dim3(64 * 2 * kGemvWaves), 0, s, g);
			return true;
		}
	}
	switch (cpw) {
#define X(W) \
	case W: hipLaunchKernelGGL((k_gemv_pk<MB, NT, W, EPI>), dim3(grid), dim3(256), 0, s, g); return true;
		X(1) X(2) X(3) X(4) X(7) X(8)
#undef X
	}
	return false;
}

template <int MB, int NT>
static bool launch_pk_epi(const GemmArgs& g, int grid, int cpw, hipStream_t s) {
	switch (pk_epi(g)) {
		case kPkRaw: return launch_pk_nt<MB, NT, kPkRaw>(g, grid, cpw, s);
		case kPkFunnel: return launch_pk_nt<MB, NT, kPkFunnel>(g, grid, cpw, s);
		default: return launch_pk_nt<MB, NT, kPkGeneral>(g, grid, cpw, s);
	}
}

static bool launch_gemv_pk(const GemmArgs& g, hipStream_t s) {
	const int T = (g.N + 15) / 16, C = g.K / 128;
	const int nt = pk_nt(T), grid = (T + nt - 1) / nt, cpw = pk_cpw(C);
	const bool two = g.M > 16;
	switch (nt) {
#define X(N) \
	case N: return two ? launch_pk_epi<2, N>(g, grid, cpw, s) : launch_pk_epi<1, N>(g, grid, cpw, s);
		X(1) X(2) X(3) X(5) X(10)
#undef X
	}
	return false;
}

template <int MB, int NTB>
static bool launch_sk_ntb(const GemmArgs& g, const SkPlan& p, hipStream_t s) {
	const dim3 grid(p.bx, p.splits), block(64 * kSkWaves);
	switch (p.cpw) {
#define X(W) \
	case W: hipLaunchKernelGGL((k_gemv_sk<MB, NTB, W, kSkWaves>), grid, block, 0, s, g, p.cps); return true;
		X(1) X(2) X(3) X(4)
#undef X
	}
	return false;
}

static bool launch_gemv_sk(const GemmArgs& g, hipStream_t s) {
	const SkPlan p = sk_plan(g.N, g.K);
	// the caller sized its planes by gemv_raw_splits(): a launch with another count is refused
	if (p.cpw == 0 || g.splits != p.splits || !g.split_part) throw LaunchRefused{"gemv_sk: split count"};
	const bool two = g.M > 16;
	switch (p.ntb) {
#define X(N) \
	case N: return two ? launch_sk_ntb<2, N>(g, p, s) : launch_sk_ntb<1, N>(g, p, s);
		X(1) X(2) X(3) X(4) X(6) X(7) X(8)
#undef X
	}
	return false;
}

// k_gemv_head takes LM-head launches (argmax keys, no raw output) on the packed copy at M <= 32,
// K <= 4096 (at most 8 chunks per wave); SSLM_HIP_HEAD_PK=0 keeps them on the generic GEMVs
static bool head_pk_ok(const GemmArgs& g) {
	static const bool on = [] {
		const char* e = getenv("SSLM_HIP_HEAD_PK");
		return !(e && atoi(e) == 0);
	}();
	return on && g.wp && g.epi.argmax_key && !g.epi.raw_out && g.splits <= 1 && g.M >= 1 && g.M <= 32 &&
	       g.K % 128 == 0 && g.K <= 4096;
}

template <int MB>
static bool launch_gemv_head(const GemmArgs& g, hipStream_t s) {
	const int C = g.K / 128, need = (C + kGemvWaves - 1) / kGemvWaves, T = (g.N + 15) / 16;
	const int grid = std::min(T, std::max(device_cus(), (T + kHeadMaxSteps - 1) / kHeadMaxSteps));
	switch (need <= 3 ? 3 : (need <= 4 ? 4 : (need <= 7 ? 7 : 8))) {
		case 3: hipLaunchKernelGGL((k_gemv_head<MB, 3>), dim3(grid), dim3(256), 0, s, g); return true;
		case 4: hipLaunchKernelGGL((k_gemv_head<MB, 4>), dim3(grid), dim3(256), 0, s, g); return true;
		case 7: hipLaunchKernelGGL((k_gemv_head<MB, 7>), dim3(grid), dim3(256), 0, s, g); return true;
		default: hipLaunchKernelGGL((k_gemv_head<MB, 8>), dim3(grid), dim3(256), 0, s, g); return true;
	}
}

void gemm(const GemmArgs& g, hipStream_t s) {
	if (g.M <= 0 || g.N <= 0) return;
	check_gemm_outputs(g);
	if (head_pk_ok(g)) {
		if (g.M > 16 ? launch_gemv_head<2>(g, s) : launch_gemv_head<1>(g, s)) return;
	}
	if (gemv_eligible(g.M, g.K) && g.wp && g.M <= kPkMaxM && !g.epi.argmax_key) {
		if (g.splits > 1 && sk_ok(g.M, g.K, &g)) {
			if (launch_gemv_sk(g, s)) return;
		} else if (pk_ok(g)) {
			if (launch_gemv_pk(g, s)) return;
		}
	}
	if (gemv_eligible(g.M, g.K)) {
		// g.splits > 1 only as gemv_plan(M, N, K, true, raw).splits, for which the caller sized
		// split_part
		const bool raw = g.splits > 1 || g.epi.raw_out || g.epi.argmax_key;
		const GemvPlan p = gemv_plan(g.M, g.N, g.K, g.splits > 1, raw);
		if (p.wave_tile) {
			const dim3 grid((g.N + 63) / 64, p.splits), block(256);
			const size_t lds = (size_t)16 * p.cps * 128;
			if (g.wp) {
				switch (p.cpw) {
					case 2: hipLaunchKernelGGL((k_gemv_w<2, true>), grid, block, lds, s, g, p.cps); break;
					case 6: hipLaunchKernelGGL((k_gemv_w<6, true>), grid, block, lds, s, g, p.cps); break;
					case 9: hipLaunchKernelGGL((k_gemv_w<9, true>), grid, block, lds, s, g, p.cps); break;
					default: hipLaunchKernelGGL((k_gemv_w<3, true>), grid, block, lds, s, g, p.cps); break;
				}
				return;
			}
			switch (p.cpw) {
				case 2: hipLaunchKernelGGL((k_gemv_w<2, false>), grid, block, lds, s, g, p.cps); break;
				case 6: hipLaunchKernelGGL((k_gemv_w<6, false>), grid, block, lds, s, g, p.cps); break;
				case 9: hipLaunchKernelGGL((k_gemv_w<9, false>), grid, block, lds, s, g, p.cps); break;
				default: hipLaunchKernelGGL((k_gemv_w<3, false>), grid, block, lds, s, g, p.cps); break;
			}
			return;
		}
		const int mblocks = (g.M + 15) / 16;
		if (gemv_persistent_ok(g)) {
			if (mblocks == 1) launch_gemv_p<1>(g, s);
			else launch_gemv_p<2>(g, s);
			return;
		}
		if (p.tpw == 2 && mblocks == 1) {
			launch_gemv<1, 2>(g, p, s);
		} else if (p.tpw == 2 && mblocks == 2) {
			launch_gemv<2, 2>(g, p, s);
		} else {
			switch (mblocks) {
				case 1: launch_gemv<1, 1>(g, p, s); break;
				case 2: launch_gemv<2, 1>(g, p, s); break;
				case 3: launch_gemv<3, 1>(g, p, s); break;
				default: launch_gemv<4, 1>(g, p, s); break;
			}
		}
		return;
	}
	bool lora = false;
	for (int i = 0; i < g.epi.nseg; ++i) lora = lora || g.epi.seg[i].lora_b;
	if (wide_gemm_ok(g)) {
		const int tiles = ((g.M + kWideBM - 1) / kWideBM) * ((g.N + kWideBN - 1) / kWideBN);
		hipLaunchKernelGGL(k_gemm_wide, dim3(tiles), dim3(256), 0, s, g);
		return;
	}
	if (!lora && !g.epi.argmax_key && prefill_mfma_k(g.K) && (g.epi.raw_out || g.N % 16 == 0)) {
		// g.splits > 1 only as prefill_plan(M, N, K, true).splits, sized by the caller
		// a raw single-plane launch of a narrow shape takes the 64 x 64-tile kernel
		if (g.epi.raw_out && g.splits <= 1 && prefill_plan(g.M, g.N, g.K, true).narrow) {
			const int tiles = ((g.M + kNarrowTile - 1) / kNarrowTile) * ((g.N + kNarrowTile - 1) / kNarrowTile);
			hipLaunchKernelGGL(k_gemm_narrow, dim3(tiles), dim3(256), 0, s, g);
			return;
		}
		const PrefillPlan p = prefill_plan(g.M, g.N, g.K, g.splits > 1);
		const dim3 grid(p.blocks, 1, p.splits);
		if (p.bm == 256) hipLaunchKernelGGL((k_gemm_mfma<256, kPrefillStages>), grid, dim3(512), 0, s, g, p);
		else hipLaunchKernelGGL((k_gemm_mfma<128, kPrefillStages>), grid, dim3(256), 0, s, g, p);
		return;
	}
	dim3 grid((g.N + kBN - 1) / kBN, (g.M + kBM - 1) / kBM);
	hipLaunchKernelGGL(k_gemm_tiled, grid, dim3(kBlock), 0, s, g);
}

bool prefill_mfma_k(int K) { return K > 0 && K % kPBK == 0; }

// The 256 x 160-tile kernel where it takes fewer tile rounds' worth of columns than 256 x 128
// tiles (a round: 256 tiles, one per CU), for raw output or funnel segments without bias / LoRA.
bool wide_gemm_ok(const GemmArgs& g) {
	if (g.M <= 64 || g.splits > 1 || g.epi.argmax_key || !prefill_mfma_k(g.K)) return false;
	if (!g.epi.raw_out) {
		// the epilogue's fold_bounded needs |acc| <= 2^29: K <= 32768 int8 products
		if (g.N % 16 != 0 || g.epi.nseg < 1 || g.K > kWideFoldMaxK) return false;
		for (int i = 0; i < g.epi.nseg; ++i) {
			const Segment& sg = g.epi.seg[i];
			if (sg.mode != kSegFunnel || sg.bias || sg.lora_b || sg.n_begin % 16 || sg.n_end % 16) return false;
		}
	}
	const int64_t rows = (g.M + 255) / 256;
	const int64_t t128 = rows * ((g.N + kPBN - 1) / kPBN), t160 = rows * ((g.N + kWideBN - 1) / kWideBN);
	if (t128 < kPrefillTargetBlocks) return false;
	return ((t160 + 255) / 256) * kWideBN < ((t128 + 255) / 256) * kPBN;
}

PrefillPlan prefill_plan(int M, int N, int K, bool split_ok) {
	PrefillPlan p{};
	p.bm = M >= 256 ? 256 : 128;
	const int tiles = ((M + p.bm - 1) / p.bm) * ((N + kPBN - 1) / kPBN);
	const int steps = (K + kPBK - 1) / kPBK;
	p.splits = 1;
	// narrow: raw output of 64 x 64 tiles, one plane, for consumers that add raw planes.  Every
	// small tile streams its whole K of both operands, so long K (the down projection) keeps
	// the large tiles with K split into planes.
	p.narrow = split_ok && tiles < kPrefillTargetBlocks && K <= kNarrowMaxK;
	if (p.narrow) {
		p.kspan = K;
		p.blocks = tiles;
		return p;
	}
	// A long-K shape of few 256-row tiles (the down projection at 512 tokens: 24 tiles) takes
	// 128-row tiles when they still fill the chip in one round with at least two K splits: 48
	// tiles x 5 splits = 240 blocks of 14 steps against 24 x 8 = 192 blocks of 9 steps, and 5
	// raw planes for the consumer to add instead of 8 (1.5B prefill GEMM pass 1748 -> 1708 us).
	if (split_ok && tiles < kPrefillTargetBlocks && M >= 256) {
		const int t128 = ((M + 127) / 128) * ((N + kPBN - 1) / kPBN);
		const int s128 = std::min({kPrefillTargetBlocks / t128, steps / 2, kMaxRawSplits});
		if (s128 >= 2) {
			p.bm = 128;
			p.splits = s128;
			const int sp = (steps + p.splits - 1) / p.splits;
			p.kspan = sp * kPBK;
			p.splits = (K + p.kspan - 1) / p.kspan;
			p.blocks = t128;
			return p;
		}
	}
	if (split_ok && tiles < kPrefillTargetBlocks)
		p.splits = std::max(1, std::min({(kPrefillTargetBlocks + tiles - 1) / tiles, steps / 2, kMaxRawSplits}));
	const int steps_per = (steps + p.splits - 1) / p.splits;
	p.kspan = steps_per * kPBK;
	p.splits = (K + p.kspan - 1) / p.kspan;
	p.blocks = tiles;
	return p;
}

void embed(const int32_t* tokens, int M, const int8_t* embed_w, int H, int vocab, Scale site, int8_t* out_codes,
           const int32_t* out_idx, Scale* out_scale, const int32_t* scale_idx, const TokenInfo* tok,
           int32_t* status, hipStream_t s) {
	hipLaunchKernelGGL(k_embed, dim3(M), dim3(kRowBlock), 0, s, tokens, embed_w, H, vocab, site, out_codes, out_idx,
	                   out_scale, scale_idx, tok, status);
}

// Row kernels are instantiated for a set of per-thread element counts; the smallest one that
// covers the row is launched.
constexpr int kRowBS = 512;     // qkv_post, residual (decode rows of H elements)
constexpr int kRowWideMaxRows = 64;  // residual launches of at most this many rows take 1024 threads
constexpr int kActBS = 1024;    // mlp_act (rows of I elements)
constexpr int kFunnelBS = 512;  // funnel, rmsnorm
static_assert(16 * kFunnelBS >= kFunnelMaxN, "funnel instances must cover kFunnelMaxN");

#define SSLM_EPT_CASES(X) X(1) X(2) X(3) X(4) X(6) X(8) X(12) X(16)
#define SSLM_ACT_EPT_CASES(X) X(1) X(2) X(4) X(9) X(12) X(20)

static int row_ept(int n, int bs) { return (n + bs - 1) / bs; }

// Geometry is validated before any launch (row_geometry_ok at model map, argument checks at the
// test entry points); a row no instance covers is a bug, not a case to skip silently.
[[noreturn]] static void no_instance(const char* kernel, int n) {
	fprintf(stderr, "sslm_hip: no %s instance for a row of %d elements\n", kernel, n);
	throw LaunchRefused{kernel};
}

void rmsnorm(const RowNormArgs& a, int M, int H, const TokenInfo* tok, int32_t* status, int32_t layer,
             hipStream_t s) {
	const int need = row_ept(H, kFunnelBS);
#define X(E)                                                                                               \
	if (need <= E) {                                                                                       \
		hipLaunchKernelGGL((k_rmsnorm<kFunnelBS, E>), dim3(M), dim3(kFunnelBS), 0, s, a, H, tok, status, layer); \
		return;                                                                                            \
	}
	SSLM_EPT_CASES(X)
#undef X
	no_instance("rmsnorm", H);
}

void qkv_post(const QkvPostArgs& a, hipStream_t s) {
	const int need = row_ept(a.H / 2, kRowBS);
#define X(E)                                                                                          \
	if (need <= E) {                                                                                  \
		if (!a.raw.part) hipLaunchKernelGGL((k_qkv_post<kRowBS, E, 0>), dim3(a.M), dim3(kRowBS), 0, s, a); \
		else if (a.raw.splits == 1) hipLaunchKernelGGL((k_qkv_post<kRowBS, E, 1>), dim3(a.M), dim3(kRowBS), 0, s, a); \
		else hipLaunchKernelGGL((k_qkv_post<kRowBS, E, kMaxRawSplits>), dim3(a.M), dim3(kRowBS), 0, s, a); \
		return;                                                                                       \
	}
	X(1) X(2) X(4) X(8)
#undef X
	no_instance("qkv_post", a.H);
}

void slot_state_copy(const SlotCopyArgs& a, int n, bool restore, hipStream_t s) {
	const int64_t nc = (int64_t)(a.l1 - a.l0) * 2 * a.NKV * a.D / 16;
	if (a.H % 16 == 0 && a.H <= 16 * 256 && nc >= 1 && nc <= 256 * kSnapKvPer)
		hipLaunchKernelGGL(k_slot_state_copy, dim3(n), dim3(256), 0, s, a, restore ? 1 : 0);
	else
		hipLaunchKernelGGL(k_slot_state_copy_any, dim3(n), dim3(256), 0, s, a, restore ? 1 : 0);
}

void kv_commit(const QkvPostArgs& a, hipStream_t s) {
	hipLaunchKernelGGL(k_kv_commit, dim3(a.M), dim3(256), 0, s, a);
}

template <bool FUSED>
static void launch_attention(const AttnArgs& a, hipStream_t s) {
	const size_t lds = (size_t)a.cap * sizeof(int64_t);
	const int use_lds = attention_in_lds(a.cap) ? 1 : 0;
	const int groups = a.M * a.NKV, per_xcd = (groups + 7) / 8;
	const dim3 grid(per_xcd * 8 * (a.NH / a.NKV));  // see the XCD-aware order in k_attention
	const size_t dyn = use_lds ? lds : 0;
	switch (a.D) {
		case 32:
			if (use_lds) hipLaunchKernelGGL((k_attention<kBlock, 32, FUSED, true>), grid, dim3(kBlock), dyn, s, a);
			else hipLaunchKernelGGL((k_attention<kBlock, 32, FUSED, false>), grid, dim3(kBlock), dyn, s, a);
			break;
		case 64:
			if (use_lds) hipLaunchKernelGGL((k_attention<kBlock, 64, FUSED, true>), grid, dim3(kBlock), dyn, s, a);
			else hipLaunchKernelGGL((k_attention<kBlock, 64, FUSED, false>), grid, dim3(kBlock), dyn, s, a);
			break;
		case 128:
			if (use_lds) hipLaunchKernelGGL((k_attention<kBlock, 128, FUSED, true>), grid, dim3(kBlock), dyn, s, a);
			else hipLaunchKernelGGL((k_attention<kBlock, 128, FUSED, false>), grid, dim3(kBlock), dyn, s, a);
			break;
		case 256:
			if (use_lds) hipLaunchKernelGGL((k_attention<kBlock, 256, FUSED, true>), grid, dim3(kBlock), dyn, s, a);
			else hipLaunchKernelGGL((k_attention<kBlock, 256, FUSED, false>), grid, dim3(kBlock), dyn, s, a);
			break;
		default: no_instance("attention", a.D);
	}
}

void attention(const AttnArgs& a, hipStream_t s, bool one_sequence) {
	if (!one_sequence || !tiled_attention_enabled()) {
		launch_attention<false>(a, s);
		return;
	}
	const int groups = ((a.M + 15) / 16) * a.NKV, per_xcd = (groups + 7) / 8;
	const dim3 grid(per_xcd * 8 * (a.NH / a.NKV));  // see the XCD-aware order in k_attention_tiled
	// 8 waves (128 positions per step) halve the longest rows' serial chain when the grid is
	// small; with two or more blocks per CU, 4-wave blocks pack the CUs better
	// SSLM_HIP_TILED_WAVES=4 or 8 overrides the choice (read per launch; the parity tests run both)
	const char* fw = getenv("SSLM_HIP_TILED_WAVES");
	const bool wide = fw && fw[0] ? fw[0] == '8' : (int)grid.x < 2 * 256;  // MI355X: 256 CUs
	switch (a.D) {
		case 32: if (wide) hipLaunchKernelGGL((k_attention_tiled<32, 8>), grid, dim3(512), 0, s, a); else hipLaunchKernelGGL((k_attention_tiled<32, 4>), grid, dim3(256), 0, s, a); break;
		case 64: if (wide) hipLaunchKernelGGL((k_attention_tiled<64, 8>), grid, dim3(512), 0, s, a); else hipLaunchKernelGGL((k_attention_tiled<64, 4>), grid, dim3(256), 0, s, a); break;
		case 128: if (wide) hipLaunchKernelGGL((k_attention_tiled<128, 8>), grid, dim3(512), 0, s, a); else hipLaunchKernelGGL((k_attention_tiled<128, 4>), grid, dim3(256), 0, s, a); break;
		case 256: if (wide) hipLaunchKernelGGL((k_attention_tiled<256, 8>), grid, dim3(512), 0, s, a); else hipLaunchKernelGGL((k_attention_tiled<256, 4>), grid, dim3(256), 0, s, a); break;
		default: no_instance("attention", a.D);
	}
}

bool tiled_attention_enabled() {
	static const bool on = [] {
		const char* e = getenv("SSLM_HIP_TILED_ATTN");
		return !(e && e[0] == '0');
	}();
	return on;
}
// The grouped decode kernel's dynamic LDS holds the [G][cap] int32 scores; with its static LDS
// (read from the instantiation once) it must fit the CU's 160 KB, else one block per head runs.
constexpr size_t kCuLds = 160 * 1024;  // gfx950: LDS per CU (one grouped block per CU)

template <int D, int GM>
static size_t group_attention_static_lds() {
	static const size_t stat = [] {
		const void* fn = reinterpret_cast<const void*>(&k_attention_group<D, 8, GM>);
		hipFuncAttributes fa{};
		if (hipFuncGetAttributes(&fa, fn) != hipSuccess) {
			fprintf(stderr, "sslm_hip: k_attention_group attributes unavailable\n");
			throw LaunchRefused{"attention_group"};
		}
		// allow the block the rest of the CU's LDS for its scores
		if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)(kCuLds - fa.sharedSizeBytes)) != hipSuccess) {
			fprintf(stderr, "sslm_hip: k_attention_group dynamic LDS limit refused\n");
			throw LaunchRefused{"attention_group"};
		}
		return (size_t)fa.sharedSizeBytes;
	}();
	return stat;
}

// GM: the group size rounded up to 4, 8 or 16 (the softmax loops' unrolled row count); 0 when
// the group does not fit the kernel (G * D / 2 <= 512 threads for the q post-processing)
static int group_rows(int G, int D) {
	const int gm = G <= 4 ? 4 : (G <= 8 ? 8 : (G <= 16 ? 16 : 0));
	return gm && G * (D / 2) <= 512 && (D <= 64 || gm <= (D == 128 ? 8 : 4)) ? gm : 0;
}

// rows per block: the group, or its first half (the second takes the rest)
static int group_block_rows(const AttnArgs& a) {
	const int G = a.NH / a.NKV;
	return a.row_halves == 2 ? (G + 1) / 2 : G;
}

template <int D, int GM>
static bool launch_attention_group_gm(const AttnArgs& a, hipStream_t s) {
	if (a.wcap < 1 || a.wcap % 128 != 0 || !(a.row_halves == 1 || a.row_halves == 2)) return false;
	const size_t dyn = (size_t)group_block_rows(a) * (size_t)a.wcap * sizeof(int32_t);  // the [rows][wcap] int32 scores
	if (group_attention_static_lds<D, GM>() + dyn > kCuLds) return false;
	const int groups = a.M * a.NKV;
	const int grid = a.row_halves == 2 ? (groups + 7) / 8 * 16 : groups;  // see the block numbering
	hipLaunchKernelGGL((k_attention_group<D, 8, GM>), dim3(grid), dim3(512), dyn, s, a);
	return true;
}

template <int D>
static bool launch_attention_group(const AttnArgs& a, hipStream_t s) {
	switch (group_rows(group_block_rows(a), D)) {
		case 4: return launch_attention_group_gm<D, 4>(a, s);
		case 8: if constexpr (D <= 128) return launch_attention_group_gm<D, 8>(a, s); else return false;
		case 16: if constexpr (D <= 64) return launch_attention_group_gm<D, 16>(a, s); else return false;
		default: return false;
	}
}

static bool attention_prepare_rows(int D, int G);

bool attention_prepare(int D, int G) {
	for (const int rows : {G, (G + 1) / 2})
		if (!attention_prepare_rows(D, rows)) return false;
	return true;
}

static bool attention_prepare_rows(int D, int G) {
	try {
		const int gm = group_rows(G, D);
		if (D == 32 && gm == 4) (void)group_attention_static_lds<32, 4>();
		if (D == 32 && gm == 8) (void)group_attention_static_lds<32, 8>();
		if (D == 32 && gm == 16) (void)group_attention_static_lds<32, 16>();
		if (D == 64 && gm == 4) (void)group_attention_static_lds<64, 4>();
		if (D == 64 && gm == 8) (void)group_attention_static_lds<64, 8>();
		if (D == 64 && gm == 16) (void)group_attention_static_lds<64, 16>();
		if (D == 128 && gm == 4) (void)group_attention_static_lds<128, 4>();
		if (D == 128 && gm == 8) (void)group_attention_static_lds<128, 8>();
		if (D == 256 && gm == 4) (void)group_attention_static_lds<256, 4>();
	} catch (const LaunchRefused&) {
		return false;
	}
	return true;
}

int group_row_halves(int M, int NKV, int G) {
	const char* e = getenv("SSLM_HIP_GROUP_HALVES");  // read per call, as below
	if (e && e[0]) return e[0] == '2' && G >= 2 ? 2 : 1;
	// two blocks per group while that still leaves no CU with two
	return G >= 2 && 2 * M * NKV <= 256 ? 2 : 1;
}

bool grouped_attention_chosen(int M, int NKV, int64_t cap) {
	// read per call: decode graphs carry the choice in their key, so a change takes effect at once
	const char* e = getenv("SSLM_HIP_GROUPED_ATTN");
	if (e && e[0]) return e[0] != '0';
	// a block per (token, KV head) fills enough CUs only for batches of long rows; short rows and
	// small batches run faster as one block per query head
	return M * NKV >= 64 && cap >= 1024;
}

void attention_decode(const AttnArgs& a, hipStream_t s) {
	if (grouped_attention_chosen(a.M, a.NKV, a.cap)) {
		bool done = false;
		switch (a.D) {
			case 32: done = launch_attention_group<32>(a, s); break;
			case 64: done = launch_attention_group<64>(a, s); break;
			case 128: done = launch_attention_group<128>(a, s); break;
			case 256: done = launch_attention_group<256>(a, s); break;
			default: break;
		}
		if (done) return;  // else the shape does not fit the grouped kernel: one block per head
	}
	launch_attention<true>(a, s);
}

void funnel(const FunnelArgs& a, hipStream_t s) {
	const int need = row_ept(a.N, kFunnelBS);
#define X(E)                                                                               \
	if (need <= E) {                                                                       \
		hipLaunchKernelGGL((k_funnel<kFunnelBS, E>), dim3(a.M), dim3(kFunnelBS), 0, s, a); \
		return;                                                                            \
	}
	SSLM_EPT_CASES(X)
#undef X
	no_instance("funnel", a.N);
}

void residual_norm(const ResidualArgs& a, hipStream_t s) {
	// decode launches (a few rows, one block each on otherwise idle CUs) of long rows: 1024
	// threads per row, so each thread's share of the row and of its raw planes is half as long
	// (measured: 7B rows of 3584 gain, 1.5B rows of 1536 at 3 per thread lose)
	if (a.M <= kRowWideMaxRows && row_ept(a.H, kRowBS) > 4) {
		const int need1k = row_ept(a.H, 1024);
#define X(E)                                                                                               \
	if (need1k <= E) {                                                                                     \
		if (!a.raw.part) hipLaunchKernelGGL((k_residual_norm<1024, E, 0>), dim3(a.M), dim3(1024), 0, s, a); \
		else if (a.raw.splits == 1) hipLaunchKernelGGL((k_residual_norm<1024, E, 1>), dim3(a.M), dim3(1024), 0, s, a); \
		else hipLaunchKernelGGL((k_residual_norm<1024, E, kMaxRawSplits>), dim3(a.M), dim3(1024), 0, s, a); \
		return;                                                                                            \
	}
		X(1) X(2) X(4) X(8)
#undef X
	}
	const int need = row_ept(a.H, kRowBS);
#define X(E)                                                                                               \
	if (need <= E) {                                                                                       \
		if (!a.raw.part) hipLaunchKernelGGL((k_residual_norm<kRowBS, E, 0>), dim3(a.M), dim3(kRowBS), 0, s, a); \
		else if (a.raw.splits == 1) hipLaunchKernelGGL((k_residual_norm<kRowBS, E, 1>), dim3(a.M), dim3(kRowBS), 0, s, a); \
		else hipLaunchKernelGGL((k_residual_norm<kRowBS, E, kMaxRawSplits>), dim3(a.M), dim3(kRowBS), 0, s, a); \
		return;                                                                                            \
	}
	SSLM_EPT_CASES(X)
#undef X
	no_instance("residual_norm", a.H);
}

void mlp_act(const ActArgs& a, hipStream_t s) {
	const int need = row_ept(a.I, kActBS);
#define X(E)                                                                                         \
	if (need <= E) {                                                                                 \
		if (!a.raw.part) hipLaunchKernelGGL((k_mlp_act<kActBS, E, 0>), dim3(a.M), dim3(kActBS), 0, s, a); \
		else if (a.raw.splits == 1) hipLaunchKernelGGL((k_mlp_act<kActBS, E, 1>), dim3(a.M), dim3(kActBS), 0, s, a); \
		else hipLaunchKernelGGL((k_mlp_act<kActBS, E, kMaxRawSplits>), dim3(a.M), dim3(kActBS), 0, s, a); \
		return;                                                                                      \
	}
	SSLM_ACT_EPT_CASES(X)
#undef X
	no_instance("mlp_act", a.I);
}

constexpr int kActSliceBS = 256;
constexpr int kActSliceMax = 1280;  // columns per slice: EPT <= 5

bool mlp_act_sliced_ok(const ActArgs& a) {
	return !a.raw.part && a.M <= kMaxSlicedActRows && a.prod && a.act_maxpart && a.gu_scale &&
	       a.I <= kMaxActSlices * kActSliceMax;
}

void mlp_act_sliced(const ActArgs& a, hipStream_t s) {
	const int S = std::max(1, std::min(kMaxActSlices, (a.I + kActSliceMax - 1) / kActSliceMax));
	const int per = ((a.I + S - 1) / S + 15) / 16 * 16;
	const int ept = (per + kActSliceBS - 1) / kActSliceBS;
	const dim3 grid(a.M, (a.I + per - 1) / per);
#define X(E)                                                                                                  \
	if (ept <= E) {                                                                                           \
		hipLaunchKernelGGL((k_mlp_act_s1<kActSliceBS, E>), grid, dim3(kActSliceBS), 0, s, a, per);             \
		hipLaunchKernelGGL((k_mlp_act_s2<kActSliceBS, E>), grid, dim3(kActSliceBS), 0, s, a, per);             \
		return;                                                                                               \
	}
	X(1) X(2) X(3) X(4) X(5)
#undef X
	no_instance("mlp_act_sliced", a.I);
}

bool row_geometry_ok(int H, int I, int NKV, int D) {
	return H <= 16 * kRowBS && H <= 16 * kFunnelBS && I <= 20 * kActBS && NKV * D <= 4 * kRowBS && H / 2 <= 8 * kRowBS &&
	       (D == 32 || D == 64 || D == 128 || D == 256);
}

void lora_u(const LoraUArgs& a, hipStream_t s) { hipLaunchKernelGGL(k_lora_u, dim3(a.M, a.nproj), dim3(kBlock), 0, s, a); }

void topk_candidates(const int32_t* logits, int V, int M, const uint8_t* const* mask_page, int k, int2* out,
                     hipStream_t s) {
	if (M <= 0) return;
	hipLaunchKernelGGL(k_topk, dim3(M), dim3(kTopKBlock), 0, s, logits, V, mask_page, k, out);
}

void stream_read(const void* p, int64_t bytes, int* sink, hipStream_t s) {
	const int64_t nvec = bytes / 16;
	const int blocks = (int)std::max<int64_t>(1, std::min<int64_t>(1024, (nvec + 1023) / 1024));
	hipLaunchKernelGGL(k_stream_read, dim3(blocks), dim3(256), 0, s, (const v4i*)p, nvec, sink);
}

void debug_gather(const int8_t* src, const Scale* ssrc, const int32_t* idx, int n, int M, int8_t* dst, Scale* sdst,
                  int ld, hipStream_t s) {
	if (M > 0) hipLaunchKernelGGL(k_debug_gather, dim3(M), dim3(256), 0, s, src, ssrc, idx, n, dst, sdst, ld);
}

void argmax_finalize(const unsigned long long* keys, int ntiles, int M, int32_t* out_tokens, hipStream_t s) {
	hipLaunchKernelGGL(k_argmax_finalize, dim3(M), dim3(kRowBlock), 0, s, keys, ntiles, out_tokens);
}

}  // namespace sslm_launch
