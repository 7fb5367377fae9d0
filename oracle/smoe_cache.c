/* oracle/smoe_cache.c - TEST INFRASTRUCTURE ONLY (the CPU checker; never linked into the product).
 *
 * The expert tier's lists and one expert on a blob, restated for the checks of smoe_expert_group,
 * smoe_expert_grouped and the verify window (stratametal_amd/csrc/smoe_cache.hip, smoe_api.cpp).
 *
 *   - or_expert_group: the hit/miss split and the grouping of routed entries by expert (the contract of the
 *     reference's moe_hit_select / moe_hit_select_multi / moe_group_resident,
 *     include/strata/kernels/s2_expert_grouped.hpp:92-112, whose kernels are not in the reference tree; the order
 *     is this library's: groups in ascending expert id, entries and misses in ascending routing index).  Pinned by
 *     the tests' independent statements of the same lists (a sort of the hit indices by (expert, index)) and by
 *     the invariants a split must keep (every entry exactly once, counts, per-group expert).
 *   - or_expert_dev: one routed expert on a blob [gate rows | up rows | down rows] (NativeExpertLayout,
 *     include/strata/kernels/iq_kernels.hpp:56-65) under the decode contract: the same chain the block's decode
 *     oracle runs for a routed pair (expert_chain in smoe_oracle.c), so it is pinned by that oracle's checks and
 *     by the tests comparing it with or_moe_decode_dev's pair rows.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "smoe_oracle.h"

int or_expert_group(const int32_t* ids, int n, int kpt, int n_expert, const uint8_t* resident, int32_t* grp_expert,
                    int32_t* grp_start, int32_t* ent_dst, int32_t* ent_tok, int32_t* miss_dst, int32_t* counts) {
    if (n < 0 || kpt < 1 || n_expert < 1) return -1;
    int32_t* cnt = (int32_t*)calloc((size_t)n_expert, sizeof(int32_t));
    int32_t* next = (int32_t*)malloc(sizeof(int32_t) * (size_t)n_expert);
    if (!cnt || !next) {
        free(cnt);
        free(next);
        return -1;
    }
    int n_miss = 0;
    for (int i = 0; i < n; ++i) {
        const int e = ids[i];
        if (e >= 0 && e < n_expert && resident[e]) cnt[e]++;
    }
    int n_groups = 0, at = 0;
    for (int e = 0; e < n_expert; ++e) {
        next[e] = at;
        if (cnt[e] > 0) {
            grp_expert[n_groups] = e;
            grp_start[n_groups] = at;
            ++n_groups;
            at += cnt[e];
        }
    }
    grp_start[n_groups] = at;
    for (int i = 0; i < n; ++i) {
        const int e = ids[i];
        if (e >= 0 && e < n_expert && resident[e]) {
            const int pos = next[e]++;
            ent_dst[pos] = i;
            ent_tok[pos] = i / kpt;
        } else {
            miss_dst[n_miss++] = i;
        }
    }
    counts[0] = n_groups;
    counts[1] = at;
    counts[2] = n_miss;
    counts[3] = 0;
    free(cnt);
    free(next);
    return 0;
}
