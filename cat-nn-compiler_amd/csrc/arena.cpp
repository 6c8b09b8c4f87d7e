// First-fit arena placement with aliased lifetimes.  Host-only.
//
// Same algorithm as schedule::place_arena (crates/catnn-compile/src/schedule.rs:79-116),
// kept alike on purpose so a plan computed here is the plan the reference's
// scheduler would compute for the same requests:
//   * requests are visited in ascending (live_from, −bytes) order, ties in
//     input order (Rust's sort_by_key is stable);
//   * each goes to the lowest offset below which it fits among the already
//     placed buffers whose inclusive lifetimes overlap its own
//     (lifetimes_overlap, schedule.rs:118-120), scanning those intervals in
//     ascending start order;
//   * exceeding the cap is an error naming the buffer (schedule.rs:101-105).
// arena_conflict restates schedule.rs:123-136.
#include <algorithm>
#include <cstring>
#include <numeric>
#include <string>
#include <vector>

#include "arena.hpp"
#include "common.hpp"

namespace catnn {

static bool lifetimes_overlap(uint64_t a0, uint64_t a1, uint64_t b0, uint64_t b1) {
    return a0 <= b1 && b0 <= a1;
}

std::vector<ArenaAlloc> place_arena(const std::vector<BufferReq> &reqs, uint64_t cap) {
    std::vector<size_t> order(reqs.size());
    std::iota(order.begin(), order.end(), 0);
    std::stable_sort(order.begin(), order.end(), [&](size_t a, size_t b) {
        if (reqs[a].live_from != reqs[b].live_from) return reqs[a].live_from < reqs[b].live_from;
        return reqs[a].bytes > reqs[b].bytes;
    });
    std::vector<ArenaAlloc> placed;
    placed.reserve(reqs.size());
    std::vector<std::pair<uint64_t, uint64_t>> forbidden;
    for (size_t i : order) {
        const BufferReq &r = reqs[i];
        forbidden.clear();
        for (const ArenaAlloc &p : placed)
            if (lifetimes_overlap(p.live_from, p.live_to, r.live_from, r.live_to))
                forbidden.emplace_back(p.offset, p.offset + p.bytes);
        std::stable_sort(forbidden.begin(), forbidden.end(),
                         [](const auto &a, const auto &b) { return a.first < b.first; });
        uint64_t cursor = 0;
        bool chosen = false;
        uint64_t off = 0;
        for (const auto &f : forbidden) {
            if (f.first >= cursor + r.bytes) {
                off = cursor;
                chosen = true;
                break;
            }
            cursor = std::max(cursor, f.second);
        }
        if (!chosen) off = cursor;
        const uint64_t end = off + r.bytes;
        if (end < off || end > cap)
            fail(CATNN_ERR_FIBRATION, "buffer arena overflow: " + r.id + " needs " +
                                          std::to_string(r.bytes) + " B at t=" +
                                          std::to_string(r.live_from) + ".." +
                                          std::to_string(r.live_to) + " (cap " +
                                          std::to_string(cap) + ")");
        placed.push_back(ArenaAlloc{r.id, r.bytes, off, r.live_from, r.live_to});
    }
    return placed;
}

bool arena_conflict(const std::vector<ArenaAlloc> &a, size_t *i_out, size_t *j_out) {
    for (size_t i = 0; i < a.size(); ++i)
        for (size_t j = i + 1; j < a.size(); ++j)
            if (lifetimes_overlap(a[i].live_from, a[i].live_to, a[j].live_from, a[j].live_to)) {
                const uint64_t a1 = a[i].offset + a[i].bytes, b1 = a[j].offset + a[j].bytes;
                if (a[i].offset < b1 && a[j].offset < a1) {
                    if (i_out) *i_out = i;
                    if (j_out) *j_out = j;
                    return true;
                }
            }
    return false;
}

}  // namespace catnn

using namespace catnn;

extern "C" {

int catnn_place_arena(const catnn_buffer_req *reqs, int32_t n, uint64_t cap,
                      catnn_arena_alloc *out) {
    return guard([&] {
        CATNN_REQUIRE(n >= 0 && (n == 0 || (reqs && out)), CATNN_ERR_INVALID_ARGUMENT,
                      "place_arena: null argument");
        std::vector<BufferReq> v;
        v.reserve((size_t)n);
        for (int32_t i = 0; i < n; ++i) {
            CATNN_REQUIRE(reqs[i].id, CATNN_ERR_INVALID_ARGUMENT, "place_arena: null id");
            CATNN_REQUIRE(std::strlen(reqs[i].id) < CATNN_ID_CAP, CATNN_ERR_INVALID_ARGUMENT,
                          std::string("place_arena: id longer than 127 bytes: ") + reqs[i].id);
            v.push_back(BufferReq{reqs[i].id, reqs[i].bytes, reqs[i].live_from, reqs[i].live_to,
                                  reqs[i].checkpoint != 0});
        }
        std::vector<ArenaAlloc> placed = place_arena(v, cap);
        for (size_t i = 0; i < placed.size(); ++i) {
            std::memset(out[i].id, 0, CATNN_ID_CAP);
            std::strncpy(out[i].id, placed[i].id.c_str(), CATNN_ID_CAP - 1);
            out[i].bytes = placed[i].bytes;
            out[i].offset = placed[i].offset;
            out[i].live_from = placed[i].live_from;
            out[i].live_to = placed[i].live_to;
        }
    });
}

int catnn_arena_conflict(const catnn_arena_alloc *allocs, int32_t n, int32_t *conflict, int32_t *i,
                         int32_t *j) {
    return guard([&] {
        CATNN_REQUIRE(conflict && n >= 0 && (n == 0 || allocs), CATNN_ERR_INVALID_ARGUMENT,
                      "arena_conflict: null argument");
        std::vector<ArenaAlloc> v;
        for (int32_t k = 0; k < n; ++k)
            v.push_back(ArenaAlloc{allocs[k].id, allocs[k].bytes, allocs[k].offset,
                                   allocs[k].live_from, allocs[k].live_to});
        size_t a = 0, b = 0;
        const bool c = arena_conflict(v, &a, &b);
        *conflict = c ? 1 : 0;
        if (i) *i = c ? (int32_t)a : -1;
        if (j) *j = c ? (int32_t)b : -1;
    });
}

}  // extern "C"
