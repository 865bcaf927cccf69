// Host-only check of the small-batch planner (plan_mb in
// xinfer_amd/csrc/gemv_mb_int4.hip) over random shapes: every descriptor gets
// between one range and one range per tile, the ranges sum to the plan's
// count, no range holds more tiles than the LDS result area was sized for,
// the grid is ranges x k-slices, the LDS request fits a CU, and a plan that
// splits K fits the stream's split-K slot (partials and counters).  Built and
// run by tests/test_plan_invariants.py; no GPU is touched (the planner's
// device queries are replaced below by a 256-CU stand-in).
#include "../xinfer_amd/csrc/gemv_mb_int4.hip"
namespace xhip_host {
int num_cus() { return 256; }
int launch_status() { return 0; }
bool gemv_stages_x(int64_t M, int64_t K) { return K <= 6144; }  // decides only M = 2
bool splitk_slot(hipStream_t, float**, size_t*, uint32_t**, int*) { return false; }
}
constexpr size_t kCap = (size_t)1 << 20;  // the slot sizes of scratch.hip
constexpr int kCnt = 4096;
#include <cstdio>
#include <random>
template <int EPI>
int check(std::mt19937_64& rng, int iters) {
    int bad = 0, planned = 0;
    for (int it = 0; it < iters; ++it) {
        MbParams p = {};
        const int nd = EPI == MB_PLAIN ? 1 + (int)(rng() % 4) : 1;
        for (int i = 0; i < nd; ++i) p.d[i].N = 1 + (int)(rng() % (rng() % 2 ? 200000 : 300));
        p.ndesc = nd;
        p.M = 2 + (int)(rng() % (EPI == MB_ARGMAX ? 7 : 15));
        p.K = 128 * (1 + (int)(rng() % (rng() % 2 ? 300 : 60)));
        xhip_host::MbPlan pl;
        const bool raise = rng() % 2;
        if (!xhip_host::plan_mb<EPI, f16>(p, pl, kCap, kCnt, raise)) continue;
        ++planned;
        int64_t sum = 0;
        bool ok = pl.blocks == pl.nranges * pl.ks && pl.lds <= 160 * 1024 && pl.kw >= 1 && (pl.nw % pl.kw) == 0 &&
                  (pl.ks == 1 || (pl.ws_floats <= kCap && pl.nranges <= kCnt));
        for (int i = 0; i < nd; ++i) {
            const int t = (p.d[i].N + 15) / 16;
            const int nr = p.d[i].nr;
            ok = ok && nr >= 1 && nr <= t && (t + nr - 1) / nr <= pl.tiles_blk;
            sum += nr;
        }
        ok = ok && sum == pl.nranges && p.nranges == pl.nranges;
        if (!ok) {
            if (bad < 5) printf("BAD epi=%d M=%d K=%d nd=%d N0=%d blocks=%d ranges=%d ks=%d tiles_blk=%d kw=%d lds=%zu\n", EPI, p.M, p.K, nd, p.d[0].N, pl.blocks, pl.nranges, pl.ks, pl.tiles_blk, pl.kw, pl.lds);
            ++bad;
        }
    }
    printf("epi=%d planned %d of %d, bad %d\n", EPI, planned, iters, bad);
    return bad;
}
int main() {
    std::mt19937_64 rng(12345);
    int bad = check<MB_PLAIN>(rng, 20000) + check<MB_SWIGLU>(rng, 20000) + check<MB_ARGMAX>(rng, 20000);
    return bad ? 1 : 0;
}
