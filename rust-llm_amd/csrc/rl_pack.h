// Library-private: the host mirror's per-call result block and the plan
// query it needs. A call's results land in coherent pinned host memory, in
// one layout whatever the call's rows: every row's token, kept count and used
// flag, and its first PACK_CANDS candidates. A call whose rows all take the
// stream path (at most 64 candidates a row, outputs written once at the end)
// has its kernel write there directly; any other call writes to device
// memory and one small kernel packs the results there. Either kernel writes
// a row's results with system-scope stores and its kept count last, and the
// host polls the kept counts; only a row that keeps more than PACK_CANDS
// candidates needs a copy of the rest.
#pragma once
#include <stdint.h>

#include "rl_sampler.h"

namespace rl {

constexpr uint32_t PACK_CANDS = 64;

struct PackedCands {
    uint32_t ids[PACK_CANDS];
    float probs[PACK_CANDS];
};
// Candidate stride of the block, in 32-bit words: ids and probs of row r are
// at cands[r].ids / cands[r].probs, i.e. r * PACK_STRIDE words past row 0's.
constexpr uint64_t PACK_STRIDE = sizeof(PackedCands) / 4;

// Packs rows 0..rows-1 of device outputs into the block's arrays (device
// addresses of coherent pinned host memory): out_token/out_kept/out_used
// [rows], out_cands[rows].
int launch_pack_rows(const uint32_t *token, const uint32_t *kept, const uint8_t *used, const uint32_t *ids,
                     const float *probs, uint64_t cand_stride, uint32_t rows, uint32_t *out_token,
                     uint32_t *out_kept, uint8_t *out_used, PackedCands *out_cands, void *stream);

// Whether rows 0..rows-1 of the configured context all take the stream path.
bool rows_all_stream(const rl_sampler_ctx *ctx, uint32_t rows);

// Marks the context's calls as writing results that a host polls in host
// memory: the stream kernel then stores each row's results with system-scope
// stores, its kept count last (other callers wait on the stream instead).
void set_results_polled(rl_sampler_ctx *ctx, bool polled);

}  // namespace rl
