// l2fetch.hpp — the device side of L2Fetch (kernels.hpp): extra blocks of a latency-bound launch that bring the next
// one-token GEMV's rows into the L2 of the XCD whose blocks will read them.
#pragma once

#include "kernels.hpp"

namespace ple {

// Extra block j of f.blocks, launch-wide index `linear` (its XCD: linear % 8). Its GEMV blocks are
// b = xcd + 8 (q + Q i), q = j / 8, Q = f.blocks / 8: every GEMV block below f.gemv_blocks whose XCD is this block's
// goes to one of the XCD's Q extra blocks. A GEMV block's rows lie in one segment (segment rows are multiples of
// block_rows), so its values and its scales are two contiguous ranges, both whole 16-byte pieces on 16-byte
// boundaries (checked by the host). Each thread reads 16-byte pieces, 8 in flight, their indices clamped into the
// block's pieces (every load unconditional and in bounds).
__device__ __forceinline__ void l2_fetch(const L2Fetch f, int j, int linear) {
  const int nt = blockDim.x;
  const int xcd = linear & 7, q = j >> 3, Q = f.blocks >> 3;
  const int first = xcd + 8 * q;
  if (first >= f.gemv_blocks) return;
  const int nb = (f.gemv_blocks - first + 8 * Q - 1) / (8 * Q);  // this block's GEMV blocks
  const int cv = f.block_rows * f.row_bytes >> 4, cs = f.block_rows * f.scale_bytes >> 4, per = cv + cs;
  const int64_t total = (int64_t)nb * per;
  uint32_t acc = 0;
  for (int64_t base = threadIdx.x; base < total; base += 8 * (int64_t)nt) {
    uint4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t idx = min(base + (int64_t)u * nt, total - 1);
      const int i = (int)(idx / per), l = (int)(idx % per);
      const int b = first + 8 * Q * i;
      // the block's segment by selects (a segment index into the arrays would put the struct in scratch memory)
      int r = b * f.block_rows;
      const uint8_t *w = f.w[0], *ws = f.ws[0];
      if (f.nseg > 1 && r >= f.rows[0]) {
        r -= f.rows[0];
        w = f.w[1];
        ws = f.ws[1];
        if (f.nseg > 2 && r >= f.rows[1]) {
          r -= f.rows[1];
          w = f.w[2];
          ws = f.ws[2];
        }
      }
      const uint8_t *p = l < cv ? w + (int64_t)r * f.row_bytes + ((int64_t)l << 4)
                                : ws + (int64_t)r * f.scale_bytes + ((int64_t)(l - cv) << 4);
      v[u] = *reinterpret_cast<const uint4 *>(p);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  if (acc == 0x9e3779b9u) f.sink[threadIdx.x & 63] = acc;
}

}  // namespace ple
