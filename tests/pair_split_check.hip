// Host-only check of the row-pair kernels' division-free pair split
// (pair_split and pair_range in xinfer_amd/csrc/gemv_pair_int4.hip) over
// random launches: contiguous ranges must be [floor(g P / G),
// floor((g + 1) P / G)) for every owner g (P pairs, G owners), tiling
// [0, P) exactly, and strided owners must count the pairs g, g + G, ...
// below P.  Built and run by tests/test_plan_invariants.py; no GPU is
// touched (the launch helpers are replaced by stand-ins below).
#include "../xinfer_amd/csrc/gemv_pair_int4.hip"
namespace xhip_host {
int num_cus() { return 256; }
int launch_status() { return 0; }
}
#include <cstdio>
#include <random>

int main() {
    std::mt19937_64 rng(20261202);
    long checked = 0, bad = 0, refused = 0;
    for (int it = 0; it < 4000; ++it) {
        xhip::PairParams p = {};
        const int64_t P = 1 + (int64_t)(rng() % (rng() % 2 ? 2000000 : 5000));
        const int64_t G = 1 + (int64_t)(rng() % (rng() % 3 ? 2048 : 60000));
        p.npairs = (int32_t)P;
        if (!xhip_host::pair_split(p, G)) {
            refused += (G * G >= (1LL << 31)) ? 1 : 0;
            bad += (G * G >= (1LL << 31)) ? 0 : 1;  // refused a launch it could take
            continue;
        }
        for (int strided = 0; strided < 2; ++strided) {
            xhip::PairArgs a = {};
            a.strided = strided != 0;
            a.wq = p.wq;
            a.wr = p.wr;
            a.ws = p.ws;
            a.wm = p.wm;
            a.G = p.G;
            const int64_t step = G <= 4096 ? 1 : 1 + (int64_t)(rng() % 37);
            int64_t prev_end = 0;
            for (int64_t g = 0; g < G; g += step) {
                int q0 = 0, nh = 0;
                xhip::pair_range(a, (uint32_t)g, q0, nh);
                ++checked;
                if (strided) {
                    const int64_t want = g < P ? (P - 1 - g) / G + 1 : 0;
                    if (q0 != g || nh != want) ++bad;
                } else {
                    const int64_t b = g * P / G, e = (g + 1) * P / G;
                    if (q0 != b || nh != e - b) ++bad;
                    if (step == 1 && b != prev_end) ++bad;
                    prev_end = e;
                }
            }
            if (!strided && step == 1 && prev_end != P) ++bad;
        }
    }
    printf("pair split: %ld owner ranges checked, %ld launches refused (G^2 >= 2^31), %ld bad\n", checked,
           refused, bad);
    return bad == 0 ? 0 : 1;
}
