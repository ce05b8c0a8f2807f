// K-tile windows of the weight-gradient operands (ragged K).
//
// The weight gradient of copy g reads the group's rows [row0, row_end) of
// both operands as its K dimension, one 64-row K-tile at a time.  Each
// K-tile's loads go through a buffer descriptor rebased to the K-tile's first
// row whose size ends with the group, so rows past the group load zeros.  A
// descriptor holds a 32-bit size, but a group's rows may span more than
// 4 GiB (e.g. 300k rows of 7168 bf16 = 4.3 GB): the window is computed in 64
// bits, and its size is then clamped to what one descriptor holds.  A K-tile
// reads at most 64 rows past its base, far below the clamp, so the clamp
// never cuts a row the K-tile needs.
//
// Plain C++ (host and device), so that the arithmetic is unit-tested on the
// host.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define PMX_HOST_DEVICE __host__ __device__
#else
#define PMX_HOST_DEVICE
#endif

namespace pmx {

constexpr int kKTileRows = 64;
// Largest size one buffer descriptor holds (offsets are 32-bit, signed range).
constexpr uint64_t kMaxDescriptorBytes = 0x7fffffffull;

struct KTileWindow {
  uint64_t offset;  // bytes from the group's first row to the K-tile's first row
  uint64_t bytes;   // bytes from there to the group's end (0 past the end), clamped
};

// Window of K-tile `kt` of a group whose rows are `group_bytes` long in total,
// with `row_bytes` between consecutive rows.  `live` false (the pipeline slots
// past a block's last K-tile) gives an empty window at the group's start.
PMX_HOST_DEVICE inline KTileWindow ktile_window(uint64_t group_bytes, uint32_t row_bytes, int32_t kt, bool live) {
  const uint64_t skip = (uint64_t)(uint32_t)kt * (uint64_t)kKTileRows * row_bytes;
  KTileWindow w;
  w.offset = live ? skip : 0u;
  const uint64_t rest = (live && skip < group_bytes) ? group_bytes - skip : 0u;
  w.bytes = rest > kMaxDescriptorBytes ? kMaxDescriptorBytes : rest;
  return w;
}

}  // namespace pmx
