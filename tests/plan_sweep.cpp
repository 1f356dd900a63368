// The launch plan's bounds over a sweep of call sizes, without a GPU: for every (max_rows, rows, vocab, max_hist,
// call kind, CU count) a handle of those sizes accepts, the plan of the call must keep every chunk at least one
// 64-token step, its splits within what a row's last chunk merges, its LDS within what spx_sampler_create set (and a
// CU's 160 KiB), its LDS regions apart, and every partial and published-candidate index inside the workspace the
// handle allocates. Prints the first violation and exits 1; prints the number of plans checked otherwise.
#include <cstdio>
#include <cstdlib>

#include "spx_plan.h"

using namespace spx;

static int fails = 0;
static long checked = 0;

#define REQUIRE(cond, ...)                                                                       \
    do {                                                                                         \
        if (!(cond)) {                                                                           \
            if (fails++ < 5) {                                                                   \
                std::printf("violated: %s | ", #cond);                                           \
                std::printf(__VA_ARGS__);                                                        \
                std::printf("\n");                                                               \
            }                                                                                    \
        }                                                                                        \
    } while (0)

static void check(int cus, int max_rows, int rows, int vocab, int max_hist, bool greedy_only, bool has_hist,
                  bool has_ban) {
    const size_t limit = lds_bound(vocab, max_hist);  // what spx_sampler_create(max_vocab = vocab) sets
    if (limit > kLdsMax) return;                      // such a handle is refused
    Launch a{};
    a.rows = rows;
    a.vocab = vocab;
    plan_rows(a, cus, max_hist, greedy_only, has_hist, has_ban);
    checked++;
    const char * f = "cus %d max_rows %d rows %d vocab %d max_hist %d greedy %d hist %d ban %d";
#define ARGS cus, max_rows, rows, vocab, max_hist, (int) greedy_only, (int) has_hist, (int) has_ban
    REQUIRE(a.chunk >= 64 && a.chunk % 64 == 0, f, ARGS);
    REQUIRE((long) a.splits * a.chunk >= vocab && (long) (a.splits - 1) * a.chunk < vocab, f, ARGS);  // none empty
    REQUIRE(a.splits >= 1 && a.splits <= (greedy_only ? kMaxSplitsGreedy : kMaxSplits), f, ARGS);
    REQUIRE(a.splits == 1 || a.chunk >= kE * a.block, f, ARGS);  // a split row's chunks hold a step of the work-group
    REQUIRE((size_t) a.lds_bytes <= limit && limit <= kLdsMax, f, ARGS);
    REQUIRE(a.nwg == rows * a.splits, f, ARGS);
    // LDS regions in order and apart
    const size_t words = (size_t) (a.chunk + 31) / 32;
    REQUIRE(a.off_ctl == 0 && a.off_red >= a.off_ctl + kCtlBytes, f, ARGS);
    REQUIRE(a.off_spec >= a.off_red + 1280, f, ARGS);
    REQUIRE(!(has_hist || has_ban) || (size_t) a.off_own >= a.off_spec + words * 4, f, ARGS);
    REQUIRE(a.own_cap >= max_hist && (a.own_cap & (a.own_cap - 1)) == 0, f, ARGS);
    REQUIRE(!has_hist || (size_t) a.off_cand >= (size_t) a.off_own + (size_t) a.own_cap * 4, f, ARGS);
    REQUIRE(a.off_cand % 16 == 0 && a.off_sort >= a.off_cand + a.cand_cap * 8, f, ARGS);
    REQUIRE(a.cand_cap >= 2 * a.block, f, ARGS);
    // 512-thread work-groups: large rows, two rows or more per CU, a whole row each, two work-groups in a CU's LDS
    if (a.block == kBlockMid)
        REQUIRE(vocab >= kBigVocab && rows >= 2 * cus && a.splits == 1 && 2 * (size_t) a.lds_bytes <= kLdsMax, f, ARGS);
    REQUIRE(a.block == (vocab >= kBigVocab ? (a.block == kBlockMid ? kBlockMid : kBlockBig) : kBlockSmall), f, ARGS);
    if (!greedy_only) {
        REQUIRE(a.off_sort + kSortCap * 8 <= a.lds_bytes, f, ARGS);
        REQUIRE(a.splits * kKeep <= kSortCap && a.splits * kKeep <= a.cand_cap, f, ARGS);  // the merge's entries
    }
    // workspace: partial (row, split) at row * splits + split; its candidates kKeep entries from there
    const long last = (long) (rows - 1) * a.splits + (a.splits - 1);
    REQUIRE((size_t) (last + 1) * sizeof(Partial) <= ws_partials(max_rows), f, ARGS);
    if (!greedy_only) REQUIRE((size_t) (last + 1) * kKeep * 8 <= ws_cands(max_rows), f, ARGS);
    REQUIRE((size_t) rows * 4 <= ws_counters(max_rows) && (size_t) rows * sizeof(Pending) <= ws_pending(max_rows), f,
            ARGS);
    // the resolving kernel after a sampling launch
    if (!greedy_only) {
        Launch r{};
        plan_resolve(r, a, max_hist);
        REQUIRE((size_t) r.lds_bytes <= limit, f, ARGS);
        REQUIRE((size_t) r.off_own >= r.off_spec + (size_t) (vocab + 31) / 32 * 4, f, ARGS);
        REQUIRE((size_t) r.off_cand >= (size_t) r.off_own + (size_t) r.own_cap * 4, f, ARGS);
        const size_t wide = wide_bytes_of(r.block);
        REQUIRE(vocab >= kBigVocab ? r.block == kBlockResolve || r.block == kBlockResolveNarrow : r.block == kBlockSmall,
                f, ARGS);
        // the 512-thread layout only where the 1024-thread one would not have fit
        if (r.block == kBlockResolveNarrow) REQUIRE((size_t) r.off_cand + wide_bytes_of(kBlockResolve) > kLdsMax, f, ARGS);
        REQUIRE((size_t) r.off_cand + wide <= (size_t) r.lds_bytes, f, ARGS);
        REQUIRE(r.off_sort >= r.off_cand + 2 * kKeep * 8 && r.off_sort + 3 * 1024 <= r.lds_bytes, f, ARGS);
    }
#undef ARGS
}

int main() {
    // handles create accepts: every history up to 16384 ids at the 151936-token vocabulary (the resolving kernel's
    // narrower layout where the 1024-thread one does not fit), and the 1024-thread layout up to 8192 ids
    for (int max_hist : {0, 2048, 8192, 16384}) {
        if (lds_bound(151936, max_hist) > kLdsMax) {
            fails++;
            std::printf("refused: vocab 151936 max_hist %d\n", max_hist);
        }
        Launch a{}, r{};
        a.vocab = 151936;
        plan_resolve(r, a, max_hist);
        if ((max_hist <= 8192) != (r.block == kBlockResolve)) {
            fails++;
            std::printf("resolving block %d at max_hist %d\n", r.block, max_hist);
        }
    }
    const int cus_list[] = {256, 80, 304, 1};
    const int rows_list[] = {1, 2, 3, 4, 7, 16, 63, 64, 65, 85, 128, 255, 256, 257, 341, 480, 512, 1000, 1024, 2048, 4096};
    const int vocab_list[] = {1, 2, 31, 63, 64, 65, 100, 1000, 2048, 3072, 4096, 4097, 12288, 15000, 16000, 16383,
                              16384, 16385, 32768, 65536, 100000, 151936, 152064, 262144, 1 << 20};
    const int hist_list[] = {0, 1, 15, 128, 1000, 4096, 8192, 16384};
    for (int cus : cus_list)
        for (int rows : rows_list)
            for (int vocab : vocab_list)
                for (int max_hist : hist_list)
                    for (int kind = 0; kind < 6; kind++) {
                        const bool greedy_only = kind == 5;
                        const bool has_hist = max_hist > 0 && (kind & 1);
                        const bool has_ban = kind & 2;
                        for (int max_rows : {rows, 2 * rows + 1})
                            check(cus, max_rows, rows, vocab, max_hist, greedy_only, has_hist, has_ban);
                    }
    if (fails) {
        std::printf("%d violations in %ld plans\n", fails, checked);
        return 1;
    }
    std::printf("%ld plans within bounds\n", checked);
    return 0;
}
