// Host-only check of the launch wrappers' guards (no GPU needed): a GEMM launch without a complete
// output and row launches that no kernel instance covers must throw sslm_launch::LaunchRefused
// before anything is enqueued.  Linked against libsslm_hip.so; prints "ok" on success.
#include <cstdio>

#include "../superslm_amd/csrc/kernels.h"

using namespace sslm_launch;

template <typename F>
static bool refuses(F&& f) {
	try {
		f();
	} catch (const LaunchRefused&) {
		return true;
	}
	return false;
}

int main() {
	int bad = 0;
	auto expect = [&](bool ok, const char* what) {
		if (!ok) {
			printf("FAIL %s\n", what);
			++bad;
		}
	};
	GemmArgs g{};
	g.M = 16;
	g.N = 256;
	g.K = 1024;
	g.lda = 1024;
	expect(refuses([&] { gemm(g, nullptr); }), "gemm without any output");
	g.epi.nseg = 1;
	g.epi.seg[0].n_begin = 0;
	g.epi.seg[0].n_end = 128;  // does not cover N
	int32_t f[4];
	int32_t fold[12];
	g.epi.seg[0].out = f;
	g.epi.seg[0].fold = fold;
	expect(refuses([&] { gemm(g, nullptr); }), "gemm whose segments stop short of N");
	g.epi.seg[0].n_end = 256;
	g.epi.seg[0].fold = nullptr;
	expect(refuses([&] { gemm(g, nullptr); }), "gemm segment without fold parameters");
	g.epi.seg[0].fold = fold;
	g.epi.seg[0].n_begin = 16;
	expect(refuses([&] { gemm(g, nullptr); }), "gemm segments not starting at column 0");
	g.epi.nseg = kMaxSeg + 1;
	expect(refuses([&] { gemm(g, nullptr); }), "gemm with too many segments");

	RowNormArgs rn{};
	expect(refuses([&] { rmsnorm(rn, 1, 1 << 20, nullptr, nullptr, 0, nullptr); }), "rmsnorm row too long");
	FunnelArgs fa{};
	fa.M = 1;
	fa.N = 1 << 20;
	expect(refuses([&] { funnel(fa, nullptr); }), "funnel row too long");
	ResidualArgs ra{};
	ra.M = 1;
	ra.H = 1 << 20;
	expect(refuses([&] { residual_norm(ra, nullptr); }), "residual row too long");
	ActArgs aa{};
	aa.M = 1;
	aa.I = 1 << 22;
	expect(refuses([&] { mlp_act(aa, nullptr); }), "mlp_act row too long");
	AttnArgs at{};
	at.M = 1;
	at.NH = 1;
	at.NKV = 1;
	at.D = 48;
	at.cap = 16;
	expect(refuses([&] { attention_decode(at, nullptr); }), "attention head_dim without an instance");
	QkvPostArgs qa{};
	qa.M = 1;
	qa.H = 1 << 20;
	expect(refuses([&] { qkv_post(qa, nullptr); }), "qkv_post row too long");
	if (bad) return 1;
	printf("ok\n");
	return 0;
}
