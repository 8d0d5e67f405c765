// rkv_decode_rows32.hip -- launches of the paged Q8_0 flash-decode kernel
// (rkv_decode_kernel.h) for 17..32 query rows per kv head (e.g. 4 draft rows
// x 8 query heads per kv head in the causal verify): two waves per
// workgroup sharing the K/V tiles, 16 rows each.
#include "rkv_decode_kernel.h"

namespace rkv {

// Two waves per workgroup, 16 rows (two 8-row n-tiles) each.
hipError_t launch_decode_rows32(const DecodeLaunch &d, hipStream_t s) {
  const bool three = d.stages != 2;
  if (d.g.head_dim == 256)
    return three ? launch_decode_t<256, 2, 3, 2>(d, s) : launch_decode_t<256, 2, 2, 2>(d, s);
  return three ? launch_decode_t<128, 2, 3, 2>(d, s) : launch_decode_t<128, 2, 2, 2>(d, s);
}

}  // namespace rkv
