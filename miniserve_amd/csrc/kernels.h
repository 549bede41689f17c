// Host-side launch interface shared by the msattn translation units.
#pragma once

#include "common.h"
#include "merge_slots.h"
#include "split_kernel.h"

namespace msattn {

struct MergeParams {
  const int* hdr;     // workspace header written by the partials kernel
  const float* ml;
  const float* acc;
  void* out;
  int64_t rows;       // batch * q_len * H
  int batch, H, KVH, G, D;
  int max_parts;      // slots per row of the partition layout
  int64_t slots;      // (m, l) / acc slots the workspace holds: no slot at or past it is read
  // Shared-prefix partials folded in as well (npp per row at slots row * npp ..; npp = 0:
  // none), as the prefix pass of a cascade decode writes them.
  const float* pml;
  const float* pacc;
  int npp;
  int64_t pslots;     // slots of the shared-prefix source (rows * npp)
  int kind_hint;      // layout the caller knows the partials kernel used (0: partition
                      // slots), or -1: read it from the header
};

hipError_t launch_merge(const MergeParams& p, int q_dtype, hipStream_t stream, bool* supported);

struct WriteKVParams {
  void* k_cache;
  void* v_cache;
  const void* k;
  const void* v;
  const int32_t* table;
  const int32_t* starts;
  int64_t blk_stride, slot_stride, head_stride;
  int batch, tokens, KVH, D, bs, num_blocks, W;
  int start_offset;  // added to starts[b] (-1: starts are context lengths after the append)
};

hipError_t launch_write_kv(const WriteKVParams& p, int src_dtype, int dst_dtype,
                           hipStream_t stream, bool* supported);

struct GatherParams {
  const void* cache;
  const int32_t* table;
  const int32_t* lens;
  void* out;
  int64_t blk_stride, slot_stride, head_stride;
  int batch, max_ctx, KVH, D, bs, num_blocks, W;
};

hipError_t launch_gather(const GatherParams& p, int elt_bytes, hipStream_t stream);

}  // namespace msattn
