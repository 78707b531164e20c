// Per-sequence view of a batched decode call (SplitArgs::seq_starts set).
// Sequence b owns tokens [seq_starts[b], seq_starts[b+1]) of k_positions and
// page-table entries page_offsets[b] .. of page_table; its logical token t
// lives in physical page page_table[page_offsets[b] + t / page_tokens].
// Device metadata is not validated on the host (it may change between
// graph replays), so every index is clamped here to the array sizes the host
// declared: a malformed batch gives wrong numbers for that sequence but
// never reads outside k_positions, page_table or the KV pool.
#pragma once
#include <cstdint>

#include "kernels.h"

namespace kvb {

struct SeqExtent {
  uint32_t start;      // first k_positions entry
  uint32_t tokens;     // clamped token count (<= max_tokens)
  uint32_t table_off;  // first page_table entry
};

__device__ __forceinline__ SeqExtent seq_extent(const SplitArgs& a, uint32_t b) {
  uint32_t s0 = a.seq_starts[b], s1 = a.seq_starts[b + 1];
  s0 = s0 < a.total_tokens ? s0 : a.total_tokens;
  s1 = s1 < s0 ? s0 : (s1 < a.total_tokens ? s1 : a.total_tokens);
  uint32_t t = s1 - s0 < a.max_tokens ? s1 - s0 : a.max_tokens;
  uint32_t off = a.page_offsets[b];
  off = off < a.table_entries ? off : a.table_entries;
  const uint64_t cap = uint64_t(a.table_entries - off) * a.page_tokens;  // tokens the table slice can map
  if (t > cap) t = uint32_t(cap);
  return SeqExtent{s0, t, off};
}

// Rebase a batched call's arguments on sequence b: its block of row-heads in
// q, q_positions, scratch, counters and the outputs, its k_positions and
// page-table slice, and the token interval [0, T_b).  Splits past the
// sequence's own count see an empty interval and write empty partials
// (m = -inf, l = 0, n = 0), which every merge skips; the single-launch
// kernel instead ends those work-groups at once and merges only the
// sequence's own splits.
__device__ __forceinline__ void rebase_sequence(SplitArgs& a, uint32_t b) {
  const SeqExtent e = seq_extent(a, b);
  const size_t rh0 = size_t(b) * a.rows * a.q_heads;
  a.q += rh0 * a.dim;
  a.q_positions += size_t(b) * a.rows;
  a.k_positions += e.start;
  a.page_table += e.table_off;
  a.begin = 0;
  a.end = e.tokens;
  a.scratch += rh0 * a.splits * (size_t(a.dim) + 2);
  if (a.counters) a.counters += size_t(b) * a.kv_heads;
  if (a.m) a.m += rh0;
  if (a.l) a.l += rh0;
  if (a.n) a.n += rh0 * a.dim;
  if (a.out) {
    if (a.out_type == 2) a.out = static_cast<_Float16*>(a.out) + rh0 * a.dim;
    else a.out = static_cast<float*>(a.out) + rh0 * a.dim;
  }
}

}  // namespace kvb
