// Host-side arena planner types (schedule.rs:36-70 BufferReq / ArenaAlloc).
#pragma once

#include <cstdint>
#include <string>
#include <vector>

namespace catnn {

struct BufferReq {
    std::string id;
    uint64_t bytes;
    uint64_t live_from;  // inclusive
    uint64_t live_to;    // inclusive
    bool checkpoint;
};

struct ArenaAlloc {
    std::string id;
    uint64_t bytes;
    uint64_t offset;
    uint64_t live_from;
    uint64_t live_to;
};

// Raises Failure{CATNN_ERR_FIBRATION} on overflow of `cap`.
std::vector<ArenaAlloc> place_arena(const std::vector<BufferReq> &reqs, uint64_t cap);
bool arena_conflict(const std::vector<ArenaAlloc> &a, size_t *i, size_t *j);

}  // namespace catnn
