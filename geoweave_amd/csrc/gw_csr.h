// Key-major (CSR) view of a [B, T, K] position table, built by gw_kv_csr_build
// (kv_csr.hip) and consumed by the backward kernels (sparse_attn_bwd.hip,
// indexer_bwd.hip).
#pragma once

#include "gw_common.h"

namespace gw {

// Entries of one key are split into work items of at most kCsrChunk entries, so that the
// per-key reductions stay balanced when a few keys are chosen by many queries.
constexpr int kCsrChunk = 2048;

// The table (what the backward passes read) and, separately, the build's transient
// workspace (the radix sort's key/value ping-pong buffers and digit counts).
struct CsrLayout {
  int64_t nk = 0;  // keys = B * S
  size_t header = 0, count = 0, off = 0, item_off = 0, part_off = 0, item_key = 0, entries = 0, total = 0;
  size_t scratch = 0, hist = 0, raw = 0, ws_total = 0;  // offsets into the build workspace
  int64_t max_items = 0;  // upper bound of header[0]
  int64_t max_parts = 0;  // upper bound of header[1]
};

struct CsrView {
  const int* header;    // {n_items, n_parts}
  const int* off;       // [nk + 1]
  const int* item_off;  // [nk + 1]
  const int* part_off;  // [nk + 1]
  const int* item_key;  // [max_items] key of each work item
  const int2* entries;  // {t, j}
  int nk;
};

CsrLayout csr_layout(int64_t B, int64_t T, int64_t S, int64_t K);
CsrView csr_view(const void* csr, const CsrLayout& L);

// One work item of the key-major reductions.
struct CsrItem {
  int key;     // b * S + s
  int chunk;   // index of this item among the key's items
  int nchunk;  // items of this key
  int beg, end;  // entry range
  int part;    // partial-sum slot of this item (keys with nchunk > 1), else -1
};

// Decodes work item `item` (< header[0]).
__device__ __forceinline__ CsrItem csr_item(const CsrView& v, int item) {
  const int lo = v.item_key[item];
  CsrItem it;
  it.key = lo;
  it.chunk = item - v.item_off[lo];
  it.nchunk = v.item_off[lo + 1] - v.item_off[lo];
  const int b0 = v.off[lo], b1 = v.off[lo + 1];
  it.beg = min(b1, b0 + it.chunk * kCsrChunk);
  it.end = min(b1, it.beg + kCsrChunk);
  it.part = it.nchunk > 1 ? v.part_off[lo] + it.chunk : -1;
  return it;
}

}  // namespace gw
