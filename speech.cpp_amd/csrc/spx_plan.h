// spx_plan.h — the launch plan of a sampling call: work-groups per row and their size, and each kernel's LDS layout.
// Host code only (no device code), so that a plain C++ compiler builds it, and the plan's bounds can be checked
// without a GPU.
#pragma once

#include <algorithm>
#include <stddef.h>

#include "spx_internal.h"

namespace spx {

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// The LDS bytes every variant may take (a CU's share).
constexpr size_t kLdsMax = 160 * 1024;

// The kernel's LDS layout for one call: the control block, reduction scratch, the chunk's special-token words, its
// list of history tokens (a power of two of entries, at least max_hist), then the candidate buffer and the sorted
// candidates (also the radix path's histograms), which the wide path's region overlays.
inline size_t plan_lds(spx::Launch & a, int block, int chunk, bool greedy_only, bool has_hist, bool has_ban, int max_hist) {
    size_t off = 0;
    a.off_ctl = (int) off;
    off += kCtlBytes;
    a.off_red = (int) off;
    off += 1280;
    const size_t words = (size_t) (chunk + 31) / 32;
    a.off_spec = (int) off;
    if (has_hist || has_ban) off += align_up(words * 4, 16);
    size_t cap = 1;
    while (cap < (size_t) max_hist) cap *= 2;
    a.own_cap = (int) cap;
    a.off_own = (int) off;
    if (has_hist) off += cap * 4;
    // also where the merge of a row's chunks sorts up to kSortCap entries; a 512-thread work-group's first step sees
    // half the tokens a 1024-thread one's does, so its threshold starts lower and it keeps as many as that one
    a.cand_cap = block == kBlockMid ? 2 * kBlockBig : std::max(2 * block, kSortCap);
    off = align_up(off, 16);
    a.off_cand = (int) off;
    a.off_sort = (int) (off + (size_t) a.cand_cap * 8);
    if (!greedy_only) off = (size_t) a.off_sort + (size_t) kSortCap * 8;
    a.lds_bytes = (int) off;
    return off;
}

// The wide path's LDS bytes for a resolving work-group of `block` threads.
inline size_t wide_bytes_of(int block) {
    return block == kBlockResolve ? wide_lds_bytes<kBlockResolve>()
         : block == kBlockResolveNarrow ? wide_lds_bytes<kBlockResolveNarrow>() : wide_lds_bytes<kBlockSmall>();
}

// The resolving kernel's launch record from the sampling one: a whole row per work-group (its special tokens over the
// whole vocabulary), 1024 threads for large vocabularies (512 where a long history list leaves too little LDS for the
// 1024-thread wide path), and an LDS layout whose last region is the wide path's (the radix path's 2 x kKeep listed
// entries and its histograms fit there too).
inline size_t plan_resolve(spx::Launch & r, const spx::Launch & a, int max_hist) {
    r = a;
    r.block = a.vocab >= kBigVocab ? kBlockResolve : kBlockSmall;
    r.splits = 1;
    r.chunk = a.vocab;
    size_t off = 0;
    r.off_ctl = (int) off;
    off += kCtlBytes;
    r.off_red = (int) off;
    off += 1280;
    r.off_spec = (int) off;
    off += align_up((size_t) (a.vocab + 31) / 32 * 4, 16);
    size_t cap = 1;
    while (cap < (size_t) max_hist) cap *= 2;
    r.own_cap = (int) cap;
    r.off_own = (int) off;
    off += cap * 4;
    off = align_up(off, 16);
    r.off_cand = (int) off;
    r.off_sort = (int) (off + 2 * kKeep * 8);
    size_t end = std::max((size_t) r.off_sort + 3 * 1024, off + wide_bytes_of(r.block));
    if (r.block == kBlockResolve && end > kLdsMax) {
        r.block = kBlockResolveNarrow;
        end = std::max((size_t) r.off_sort + 3 * 1024, off + wide_bytes_of(r.block));
    }
    r.lds_bytes = (int) end;
    return end;
}

// Chunks per row: about one work-group of 1024 threads, or four of 256, per CU (`cus` of them); chunks of at least
// one step of the work-group (kE tokens a lane) and a multiple of 64 tokens, and few enough that the row's last chunk
// can merge them (kMaxSplits; kMaxSplitsGreedy for argmax-only calls, whose chunks publish no candidates). The
// workspace holds kMaxSplitsGreedy partials and kMaxSplits x kKeep candidates per row, so no chunk index reaches
// past its row's share. Large rows in batches of two or more per CU take 512-thread work-groups, a whole row each,
// where two of them fit a CU's LDS.
inline void plan_rows(Launch & a, int cus, int max_hist, bool greedy_only, bool has_hist, bool has_ban) {
    int block = a.vocab >= kBigVocab ? kBlockBig : kBlockSmall;
    if (block == kBlockBig && a.rows >= 2 * cus) {
        Launch probe = a;
        if (plan_lds(probe, kBlockMid, a.vocab, greedy_only, has_hist, has_ban, max_hist) <= kLdsMax / 2)
            block = kBlockMid;
    }
    const int per_cu = block == kBlockBig ? 1 : block == kBlockMid ? 2 : 4;
    const int max_splits = greedy_only ? kMaxSplitsGreedy : kMaxSplits;
    int splits = std::max(1, (per_cu * cus + a.rows - 1) / std::max(a.rows, 1));
    splits = std::min(splits, max_splits);
    splits = std::min(splits, std::max(1, a.vocab / (kE * block)));
    int chunk = (a.vocab + splits - 1) / splits;
    chunk = (int) align_up((size_t) chunk, 64);
    splits = (a.vocab + chunk - 1) / chunk;
    a.block = block;
    a.splits = splits;
    a.chunk = chunk;
    a.nwg = a.rows * splits;
    plan_lds(a, block, chunk, greedy_only, has_hist, has_ban, max_hist);
}

// The LDS a call up to these sizes can ask for: the largest history, and a chunk that is the whole vocabulary, in
// either work-group size a call may take, and the resolving kernel's.
inline size_t lds_bound(int max_vocab, int max_hist) {
    size_t lds_max = 0;
    for (int block : {kBlockBig, kBlockMid, kBlockSmall}) {
        Launch probe{};
        lds_max = std::max(lds_max, plan_lds(probe, block, max_vocab, false, max_hist > 0, true, max_hist));
    }
    Launch probe{}, res{};
    probe.vocab = max_vocab;
    return std::max(lds_max, plan_resolve(res, probe, max_hist));
}

}  // namespace spx
