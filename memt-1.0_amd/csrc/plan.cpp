// Host-side chunk plan of the packed update (no device work, no allocation).
//
// The reference builds its ChunkPlan from device boundary tensors with a
// device-to-host copy per call (models/qwen/ops/layout.py:47-109).  Here the
// caller passes host boundaries and receives the int32 tables in host
// buffers it owns, ready for one host-to-device copy:
//   * every write event [event[i], event[i+1]) is cut into ceil(len / wy)
//     chunks of at most wy tokens (a chunk never crosses an event);
//   * each chunk reads the snapshot of the read block that contains its
//     first token (the last read boundary <= tok0) and starts that block
//     when tok0 is the boundary itself;
//   * a sample's chunks start at the first chunk of the first event boundary
//     at or after the sample boundary;
//   * a chunk commits when its event does (commit_mask, default all).
// Boundaries are sorted, so each table is one forward sweep.
#include <stdint.h>

#include "../../include/memt_gdn2.h"

namespace {

bool bounds_ok(const int32_t* b, int n, int32_t first, int32_t last) {
  if (b == nullptr || n < 1 || b[0] != first || b[n - 1] != last) return false;
  for (int i = 1; i < n; ++i)
    if (b[i] < b[i - 1]) return false;
  return true;
}

}  // namespace

extern "C" {

int memt_gdn2_plan_count(const int32_t* event, int n_event, int wy_tile_tokens, int32_t* n_chunk) {
  if (n_chunk == nullptr || wy_tile_tokens < 1 || wy_tile_tokens > 64) return MEMT_GDN2_EINVAL;
  if (event == nullptr || n_event < 1 || event[0] != 0 || !bounds_ok(event, n_event, 0, event[n_event - 1]))
    return MEMT_GDN2_EINVAL;
  int64_t total = 0;
  for (int i = 0; i + 1 < n_event; ++i) total += (event[i + 1] - event[i] + wy_tile_tokens - 1) / wy_tile_tokens;
  if (total > INT32_MAX) return MEMT_GDN2_EINVAL;
  *n_chunk = (int32_t)total;
  return MEMT_GDN2_OK;
}

int memt_gdn2_plan_build(const int32_t* read, int n_read, const int32_t* sample, int n_sample,
                         const int32_t* event, int n_event, const uint8_t* commit_mask, int wy_tile_tokens,
                         int32_t n_chunk, int32_t* chunk_tok0, int32_t* chunk_len,
                         int32_t* sample_chunk_offsets, int32_t* chunk_block_ids, int32_t* chunk_flags,
                         int32_t* chunk_indices, int32_t* chunk_is_block_start, int32_t* chunk_commits) {
  int32_t count = 0;
  const int st = memt_gdn2_plan_count(event, n_event, wy_tile_tokens, &count);
  if (st != MEMT_GDN2_OK) return st;
  if (count != n_chunk) return MEMT_GDN2_EINVAL;
  const int32_t total = event[n_event - 1];
  if (!bounds_ok(read, n_read, 0, total) || !bounds_ok(sample, n_sample, 0, total)) return MEMT_GDN2_EINVAL;
  if (n_chunk > 0 && (chunk_tok0 == nullptr || chunk_len == nullptr || chunk_block_ids == nullptr ||
                      chunk_flags == nullptr))
    return MEMT_GDN2_EINVAL;
  const int wy = wy_tile_tokens;

  // chunks, their read blocks and flags
  int c = 0, blk = 0;
  for (int i = 0; i + 1 < n_event; ++i) {
    const int commit = commit_mask ? (commit_mask[i] != 0) : 1;
    int sub = 0;
    for (int32_t t0 = event[i]; t0 < event[i + 1]; t0 += wy, ++sub, ++c) {
      while (blk + 1 < n_read && read[blk + 1] <= t0) ++blk;  // last read boundary <= t0
      const int start = read[blk] == t0 ? 1 : 0;
      chunk_tok0[c] = t0;
      chunk_len[c] = event[i + 1] - t0 < wy ? event[i + 1] - t0 : wy;
      chunk_block_ids[c] = blk;
      chunk_flags[c] = start * MEMT_GDN2_CHUNK_BLOCK_START + commit * MEMT_GDN2_CHUNK_COMMIT;
      if (chunk_indices) {
        chunk_indices[2 * c] = i;
        chunk_indices[2 * c + 1] = sub;
      }
      if (chunk_is_block_start) chunk_is_block_start[c] = start;
      if (chunk_commits) chunk_commits[c] = commit;
    }
  }
  // sample offsets: chunk index of the first event boundary >= the sample boundary
  if (sample_chunk_offsets) {
    int e = 0, first = 0;  // first chunk of event boundary e
    for (int s = 0; s < n_sample; ++s) {
      while (e < n_event - 1 && event[e] < sample[s]) {
        first += (event[e + 1] - event[e] + wy - 1) / wy;
        ++e;
      }
      sample_chunk_offsets[s] = first;
    }
  }
  return MEMT_GDN2_OK;
}

}  // extern "C"
