// The Twilight union record of a KV group, and the score launch that the
// fused Twilight selection (twilight.hip) shares with the Quest selection
// (quest.hip).
#pragma once

#include "tw_common.h"

namespace tw {

// Union record of one KV group, rec_stride 32-bit words per group:
//   words [0, union_bits_words(P)): bit p (bit p % 32 of word p / 32) is set
//     when some query head of the group keeps a row of page p;
//   words [union_mask_offset(P), + union_mask_words(P)): the kept rows of
//     every page as a 16-bit mask, two pages per word (page p in bits
//     [16 * (p & 1), + 16) of word p / 2; bit i = row i of the page).
// The bitmap is whole 64-bit words and the masks start and end on 16 bytes,
// so both are read with wide loads.  16-row pages only.
__host__ __device__ __forceinline__ int union_bits_words(int P) { return 2 * ((P + 63) / 64); }
__host__ __device__ __forceinline__ int union_mask_offset(int P) { return (union_bits_words(P) + 3) & ~3; }
__host__ __device__ __forceinline__ int union_mask_words(int P) { return ((P + 1) / 2 + 3) & ~3; }
__host__ __device__ __forceinline__ int64_t union_record_words(int P) {
  return static_cast<int64_t>(union_mask_offset(P)) + union_mask_words(P);
}

// Scores of every (group, head) row for a selection kernel that follows.
struct FusedScores {
  const float* scores;   // row (g, r) at + (g * R + r) * score_stride, 16-byte aligned rows
  int64_t score_stride;
  int vec_last4;         // last float4 start inside a row (rows padded to 4)
  const uint2* tile_mm;  // [(g * R + r) * ceil(P / 64) + tile] = (max, min) score key of the tile
};

// The Quest score launch with the per-tile key ranges (quest.hip), which
// also clears every group's union record (rec, rec_stride words apart) so
// that the selection after it can OR into it, and zeroes n_counters arrival
// counters of that selection (whatever an earlier call of other sizes left
// in their words).  lengths (nullable): ragged groups as
// tw_quest_select_ragged.  workspace: tw_quest_select_workspace_size(G, R, P)
// bytes.  P <= 8192.
int fused_quest_score(const float* q, const void* page_min, const void* page_max, int dtype, int G, int R, int P,
                      int D, int64_t page_group_stride, const int32_t* lengths, int sink, int recent, int block_size,
                      void* workspace, size_t workspace_bytes, uint32_t* rec, int64_t rec_stride,
                      unsigned int* counters, int n_counters, FusedScores* out, hipStream_t stream);

}  // namespace tw
