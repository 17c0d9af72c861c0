// Library-private: the host mirror's per-call result block. After a sampling
// call, one small kernel writes every row's token, kept count, used flag and
// first PACK_CANDS candidates into host memory the device can write
// (coherent pinned memory), so the host reads a call's results after one
// stream synchronisation, with no copy per array and none per row; only a row
// that keeps more candidates needs a copy of the rest.
#pragma once
#include <stdint.h>

namespace rl {

constexpr uint32_t PACK_CANDS = 64;

struct PackedRow {
    uint32_t token, kept, used, pad;
    uint32_t ids[PACK_CANDS];
    float probs[PACK_CANDS];
};

// out: the device's address of rows PackedRow entries in coherent pinned host
// memory. Candidates are read from ids/probs rows of cand_stride entries.
int launch_pack_rows(const uint32_t *token, const uint32_t *kept, const uint8_t *used, const uint32_t *ids,
                     const float *probs, uint64_t cand_stride, uint32_t rows, PackedRow *out, void *stream);

}  // namespace rl
