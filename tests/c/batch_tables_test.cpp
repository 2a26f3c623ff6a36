// Host test of the model instance's resident block tables
// (xllms_amd/csrc/batch_tables.h): random exec patterns over a model of the
// KV index (page lists, handles reused after a release) and of the device
// rows, driven the way the general exec drives them (model_instance.cpp:
// appends record the pages they open; the batch either updates its rows in
// place or uploads all of them; a failed exec leaves the rows unknown).
// After every exec each row must hold its sequence's page ids, then -1.
//
// Planted mistakes (compile-time, in this test's model only): PLANT_DROP_UPDATES
// leaves the in-place updates unapplied, PLANT_NO_FORGET never tells the
// tables about releases and admissions; the checker must report both.
#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>

#include "batch_tables.h"

namespace {

struct Seq {
    std::vector<int32_t> pages;
    int32_t len = 0;
    bool live = false;
};

struct Model {
    int bs = 16, max_blocks = 64;
    std::vector<Seq> seqs;
    std::vector<int32_t> free_handles;  // reused last-freed first, as the index does
    int32_t next_page = 0;
    xhip::ResidentTables bt;
    std::vector<int32_t> dev;  // the device rows
    long checks = 0, updates = 0, uploads = 0;

    void forget(int32_t h) {
#ifndef PLANT_NO_FORGET
        bt.forget(h);
#else
        (void)h;
#endif
    }
    // appends n tokens; the pages they open, as (table entry, page)
    void append(int32_t h, int n, std::vector<std::pair<int32_t, int32_t>> *opened) {
        Seq &s = seqs[(size_t)h];
        for (int t = 0; t < n; ++t) {
            const int pos = s.len + t;
            if (pos % bs == 0) {
                s.pages.push_back(next_page++);
                if (opened) opened->push_back({pos / bs, s.pages.back()});
            }
        }
        s.len += n;
    }
    int32_t admit(int n) {
        int32_t h;
        if (!free_handles.empty()) {
            h = free_handles.back();
            free_handles.pop_back();
        } else {
            h = (int32_t)seqs.size();
            seqs.emplace_back();
        }
        seqs[(size_t)h] = Seq();
        seqs[(size_t)h].live = true;
        append(h, n, nullptr);
        forget(h);
        return h;
    }
    void release(int32_t h) {
        seqs[(size_t)h].live = false;
        forget(h);
        free_handles.push_back(h);
    }
};

struct ExecItem {
    int32_t seq;  // -1: admitted by the exec
    int tokens;
    bool query;
};

int g_fail = 0;

// One general exec; `fail` makes it fail after its device work was issued.
// Returns the items, admitted ones with their handles.
std::vector<ExecItem> exec(Model &m, std::vector<ExecItem> items, bool fail, std::mt19937 &rng,
                           const char *what) {
    std::vector<std::pair<int32_t, int32_t>> opened;
    std::vector<size_t> open0, nopen;
    std::vector<int32_t> len0;
    for (ExecItem &it : items) {
        open0.push_back(opened.size());
        if (it.seq < 0) {
            it.seq = m.admit(it.tokens);
            len0.push_back(-1);
        } else {
            len0.push_back(m.seqs[(size_t)it.seq].len);
            m.append(it.seq, it.tokens, &opened);
        }
        nopen.push_back(opened.size() - open0.back());
    }
    std::vector<int32_t> batch, lens, blen0;
    int width = 1;
    for (size_t k = 0; k < items.size(); ++k) {
        if (!items[k].query) continue;
        const Seq &s = m.seqs[(size_t)items[k].seq];
        batch.push_back(items[k].seq);
        lens.push_back(s.len);
        blen0.push_back(len0[k]);
        width = std::max(width, (s.len + m.bs - 1) / m.bs);
    }
    const int B = (int)batch.size();
    const bool update = m.bt.can_update(batch.data(), blen0.data(), B, width);
    int stride = 0;
    if (update) {
        stride = m.bt.stride;
        std::vector<int32_t> pairs;
        int i = 0;
        for (size_t k = 0; k < items.size(); ++k) {
            if (!items[k].query) continue;
            for (size_t j = open0[k]; j < open0[k] + nopen[k]; ++j) {
                pairs.push_back(m.bt.index(i, opened[j].first));
                pairs.push_back(opened[j].second);
            }
            ++i;
        }
        // the staging kernel; a failed exec may have stored any part of it
        const size_t n = fail ? (size_t)(rng() % (pairs.size() / 2 + 1)) : pairs.size() / 2;
#ifndef PLANT_DROP_UPDATES
        for (size_t j = 0; j < n; ++j) m.dev[(size_t)pairs[2 * j]] = pairs[2 * j + 1];
#else
        (void)n;
#endif
        m.updates++;
    } else if (B > 0) {
        stride = xhip::ResidentTables::upload_stride(width, m.max_blocks);
        std::vector<int32_t> rows((size_t)B * stride, -1);
        for (int i = 0; i < B; ++i) {
            const Seq &s = m.seqs[(size_t)batch[(size_t)i]];
            std::copy(s.pages.begin(), s.pages.end(), rows.begin() + (size_t)i * stride);
        }
        if (fail) {  // a failed upload may have stored any prefix of it
            const size_t n = rng() % (rows.size() + 1);
            m.dev.resize(std::max(m.dev.size(), rows.size()), 12345);
            std::copy(rows.begin(), rows.begin() + (long)n, m.dev.begin());
        } else {
            m.dev = rows;
        }
        m.uploads++;
    }
    if (fail) {  // the exec forgets its sequences' device state, then the rows
        for (const ExecItem &it : items) m.forget(it.seq);
    }
    if (B > 0 || fail)
        m.bt.commit(!fail, !update, batch.data(), lens.data(), B, stride, nullptr, 0, nullptr, 0, 0);
    if (fail || B == 0) return items;
    for (int i = 0; i < B; ++i) {
        const Seq &s = m.seqs[(size_t)batch[(size_t)i]];
        for (int j = 0; j < stride; ++j) {
            const int32_t want = j < (int)s.pages.size() ? s.pages[(size_t)j] : -1;
            const int32_t got = m.dev[(size_t)i * stride + j];
            m.checks++;
            if (got != want) {
                if (g_fail++ < 5)
                    std::fprintf(stderr, "%s: row %d (seq %d, %d tokens) entry %d holds %d, not %d\n",
                                 what, i, batch[(size_t)i], s.len, j, got, want);
                return items;
            }
        }
    }
    return items;
}

// A released handle reused by a K/V-only admission of the same length as the
// released sequence had: only the release / admission tells the tables.
void reuse_scenario() {
    Model m;
    std::mt19937 rng(1);
    std::vector<ExecItem> first = {{-1, 40, true}, {-1, 40, true}};
    exec(m, first, false, rng, "reuse: admit");
    const int32_t a = 0, b = 1;
    exec(m, {{a, 1, true}, {b, 1, true}}, false, rng, "reuse: step");
    exec(m, {{b, 0, false}}, false, rng, "reuse: release exec");
    m.release(b);
    // the new request takes b's handle, with b's length (41), without a query
    exec(m, {{-1, 41, false}}, false, rng, "reuse: K/V-only admission");
    exec(m, {{a, 1, true}, {b, 16, true}}, false, rng, "reuse: next step");
}

}  // namespace

int main() {
    reuse_scenario();
    for (int seed = 0; seed < 400; ++seed) {
        std::mt19937 rng((unsigned)seed);
        Model m;
        m.bs = (rng() & 1) ? 16 : 32;
        m.max_blocks = 2048 / m.bs;
        std::vector<int32_t> live;
        const int n0 = 2 + (int)(rng() % 7);
        std::vector<ExecItem> adm;
        for (int i = 0; i < n0; ++i) adm.push_back({-1, 1 + (int)(rng() % (3 * m.bs)), true});
        exec(m, adm, false, rng, "admit");
        for (int h = 0; h < (int)m.seqs.size(); ++h) live.push_back(h);
        char what[96];
        for (int step = 0; step < 60; ++step) {
            std::snprintf(what, sizeof what, "seed %d step %d", seed, step);
            const unsigned u = rng() % 100;
            auto grow = [&]() {
                static const int kGrow[] = {1, 1, 1, 2, 5, 17, 40};
                return kGrow[rng() % 7];
            };
            bool room = true;
            for (int32_t h : live) room = room && m.seqs[(size_t)h].len < 2048 - 45 - 40;
            std::vector<ExecItem> items;
            if (u < 60 && room) {  // the same batch again
                for (int32_t h : live) items.push_back({h, grow(), true});
                exec(m, items, rng() % 40 == 0, rng, what);
            } else if (u < 70 && room) {  // one request grows outside the batch
                const int32_t h = live[rng() % live.size()];
                exec(m, {{h, grow(), (rng() & 1) != 0}}, false, rng, what);
            } else if (u < 78) {  // another order
                for (size_t i = live.size(); i > 1; --i) std::swap(live[i - 1], live[rng() % i]);
            } else if (u < 86 && room) {  // a subset
                for (int32_t h : live)
                    if (rng() & 1) items.push_back({h, 1, true});
                if (!items.empty()) exec(m, items, false, rng, what);
            } else if (u < 94 && live.size() > 1) {  // a release, and maybe an admission
                const size_t k = rng() % live.size();
                const int32_t h = live[k];
                exec(m, {{h, 0, false}}, false, rng, what);
                m.release(h);
                live.erase(live.begin() + (long)k);
                if (rng() % 3) {  // (with or without a query: a K/V-only prefill)
                    const bool q = (rng() & 1) != 0;
                    const auto done =
                        exec(m, {{-1, 1 + (int)(rng() % (3 * m.bs)), q}}, false, rng, what);
                    live.insert(live.begin() + (long)(rng() % (live.size() + 1)), done[0].seq);
                }
            }
        }
        if (g_fail) break;
        if (seed == 399)
            std::printf("last seed: %ld entries checked, %ld in-place updates, %ld uploads\n",
                        m.checks, m.updates, m.uploads);
    }
    if (g_fail) {
        std::fprintf(stderr, "FAILED: %d stale rows\n", g_fail);
        return 1;
    }
    std::printf("PASSED\n");
    return 0;
}
