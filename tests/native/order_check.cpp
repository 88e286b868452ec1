// Host check of the MFMA pass kernels' workgroup order (poly-attention_amd/csrc/pa_order.h),
// built and run by tests/test_order.py.  For every grid shape below it checks that
// pa::block_map is a bijection from workgroup ids onto (unit, block) pairs, and, where the
// spread order applies, that every XCD runs the same number of heads of every batch row and
// whole GQA groups; heavy (causal) grids must dispatch each XCD's blocks by nondecreasing
// block rank, the others each unit's blocks consecutively.  With the argument "mutant" it
// checks a planted mistake instead (head and batch index swapped in the spread order), which
// must fail.
#include <cstdio>
#include <cstring>
#include <vector>

#include "pa_order.h"

static bool g_mutant = false;

static void map(int bid, int nblocks, int nblk, int heads, int group, bool heavy, int& unit,
                int& rank) {
    pa::block_map(bid, nblocks, nblk, heads, group, heavy, unit, rank);
    if (g_mutant && heads % (pa::kNumXcd * group) == 0 && unit >= 0) {
        const int b = unit / heads, h = unit % heads;  // planted: batch row taken as the head
        unit = (h % (nblocks / nblk / heads)) * heads + b;
    }
}

int main(int argc, char** argv) {
    g_mutant = argc > 1 && std::strcmp(argv[1], "mutant") == 0;
    long cases = 0;
    const int Bs[] = {1, 2, 3, 4, 5, 8};
    const int Hs[] = {1, 2, 3, 4, 6, 8, 12, 16, 24, 32, 64};
    const int Gs[] = {1, 2, 4, 8};
    const int Ns[] = {1, 2, 3, 4, 5, 7, 8, 16, 32, 64};
    for (int B : Bs)
        for (int H : Hs)
            for (int G : Gs) {
                if (H % G) continue;
                for (int nblk : Ns)
                    for (int heavy = 0; heavy < 2; ++heavy) {
                        const int units = B * H, nblocks = units * nblk;
                        std::vector<int> seen((size_t)nblocks, 0), xcd_of((size_t)units, -1);
                        std::vector<int> last_rank(pa::kNumXcd, -1);
                        for (int bid = 0; bid < nblocks; ++bid) {
                            int u = -1, r = -1;
                            map(bid, nblocks, nblk, H, G, heavy, u, r);
                            if (u < 0 || u >= units || r < 0 || r >= nblk) {
                                std::printf("FAIL range B=%d H=%d G=%d nblk=%d heavy=%d bid=%d -> (%d, %d)\n",
                                            B, H, G, nblk, heavy, bid, u, r);
                                return 1;
                            }
                            if (seen[(size_t)u * nblk + r]++) {
                                std::printf("FAIL duplicate B=%d H=%d G=%d nblk=%d heavy=%d (%d, %d)\n",
                                            B, H, G, nblk, heavy, u, r);
                                return 1;
                            }
                        }
                        const int per = nblocks / pa::kNumXcd;
                        const bool whole = nblocks % pa::kNumXcd == 0 && per % nblk == 0;
                        if (whole) {
                            // dispatch order on each XCD: hardware ids x, x + 8, ...
                            for (int x = 0; x < pa::kNumXcd; ++x) {
                                int prev_u = -1, prev_r = -1;
                                std::vector<int> done((size_t)units, 0);
                                for (int bid = x; bid < nblocks; bid += pa::kNumXcd) {
                                    int u, r;
                                    map(bid, nblocks, nblk, H, G, heavy, u, r);
                                    if (xcd_of[u] >= 0 && xcd_of[u] != x) {
                                        std::printf("FAIL unit split over XCDs B=%d H=%d nblk=%d\n", B, H, nblk);
                                        return 1;
                                    }
                                    xcd_of[u] = x;
                                    if (heavy && r < prev_r) {
                                        std::printf("FAIL heavy order B=%d H=%d nblk=%d\n", B, H, nblk);
                                        return 1;
                                    }
                                    if (!heavy && u != prev_u) {
                                        if (prev_u >= 0) done[prev_u] = 1;
                                        if (done[u]) {
                                            std::printf("FAIL unit blocks not consecutive B=%d H=%d nblk=%d\n", B, H, nblk);
                                            return 1;
                                        }
                                    }
                                    prev_u = u;
                                    prev_r = r;
                                }
                            }
                            if (H % (pa::kNumXcd * G) == 0) {
                                // every XCD: H / 8 heads of every batch row, whole GQA groups
                                for (int x = 0; x < pa::kNumXcd; ++x)
                                    for (int b = 0; b < B; ++b) {
                                        int n = 0;
                                        for (int h = 0; h < H; ++h) n += xcd_of[b * H + h] == x;
                                        if (n != H / pa::kNumXcd) {
                                            std::printf("FAIL spread B=%d H=%d G=%d nblk=%d heavy=%d: XCD %d has %d heads of row %d\n",
                                                        B, H, G, nblk, heavy, x, n, b);
                                            return 1;
                                        }
                                    }
                                for (int u = 0; u < units; ++u)
                                    if (xcd_of[u] != xcd_of[u - u % G]) {
                                        std::printf("FAIL GQA group split B=%d H=%d G=%d\n", B, H, G);
                                        return 1;
                                    }
                            }
                        }
                        ++cases;
                    }
            }
    std::printf("ok %ld\n", cases);
    return 0;
}
