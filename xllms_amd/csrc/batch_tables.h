// Host view of the block tables a model instance keeps on the device for its
// last attention batch (model_instance.cpp).  Header-only and free of HIP, so
// that the rules below are unit-tested on the host (tests/c/batch_tables_test.cpp).
//
// The device holds one row per batch position: the sequence's page ids, then
// -1, in rows of `stride` entries.  An exec whose batch is the same sequences
// in the same order, each grown since only by this exec's own appends, needs
// only the entries of the pages those appends opened (row i, entry pos /
// block_size for every appended position pos that starts a page); any other
// exec uploads every row again, with kSlack spare entries per row so that the
// following execs can keep updating in place.  A failed exec, and a release
// or an admission that reuses one of the batch's handles, drops the rows.
#pragma once

#include <stdint.h>

#include <algorithm>
#include <vector>

namespace xhip {

struct ResidentTables {
    static constexpr int kSlack = 16;

    std::vector<int32_t> seqs;  // the batch's sequence handles, in batch order
    std::vector<int32_t> len;   // tokens each row covers
    // the batch's prefix groups as the cascade takes them (appends never
    // share pages, so they change only with the batch)
    std::vector<int32_t> group, pblocks;
    int num_groups = 0;
    int stride = 0;
    bool valid = false;

    // Sequence handle `seq` was released, or reused for an admission.
    void forget(int32_t seq) {
        if (valid && std::find(seqs.begin(), seqs.end(), seq) != seqs.end()) valid = false;
    }

    // Whether an exec over `batch` (B handles, batch order) can update the
    // rows in place: len0[i] is the tokens batch[i] held before this exec's
    // appends (-1: admitted by this exec), width the entries its longest row
    // needs.
    bool can_update(const int32_t *batch, const int32_t *len0, int B, int width) const {
        if (!valid || B <= 0 || (size_t)B != seqs.size() || width > stride) return false;
        for (int i = 0; i < B; ++i)
            if (batch[i] != seqs[(size_t)i] || len0[i] != len[(size_t)i]) return false;
        return true;
    }

    // Row stride of a new upload: the widest row plus the spare entries
    // (rounded to 16), at most the model's table width unless a row needs more.
    static int upload_stride(int width, int max_blocks) {
        return std::min((width + kSlack + 15) / 16 * 16, std::max(max_blocks, width));
    }

    // The device entry of row i, table entry `entry` (a page opened by an
    // append), under the current stride.
    int32_t index(int i, int entry) const { return (int32_t)(i * stride + entry); }

    // After an exec's launches: what the device rows now hold.  ok: the exec
    // succeeded; uploaded: it uploaded every row at `new_stride`, with the
    // batch's groups.
    void commit(bool ok, bool uploaded, const int32_t *batch, const int32_t *lens, int B,
                int new_stride, const int32_t *grp, size_t ngrp, const int32_t *pbl, size_t npbl,
                int ng) {
        valid = ok;
        if (!ok) return;
        if (uploaded) {
            seqs.assign(batch, batch + B);
            stride = new_stride;
            group.assign(grp, grp + ngrp);
            pblocks.assign(pbl, pbl + npbl);
            num_groups = ng;
        }
        len.assign(lens, lens + B);
    }
};

}  // namespace xhip
