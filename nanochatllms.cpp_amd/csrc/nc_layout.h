// nc_layout.h -- HBM layouts of activation rows and weights (host + device).
//
// Activation rows ("Act", gten::ModuleDtype::adtype):
//   Q8 : [ nb*32 int8 codes | nb fp16 deltas | pad to 16 B ],  nb = ceil(cols/32)
//        (the reference's 34-byte blocks {f16 delta; i8 q[32]} split into two
//        arrays per row so the codes load as aligned 16-byte vectors)
//   F16: [ cols fp16 | pad to 16 B ]
//   F32: [ cols fp32 | pad to 16 B ]
// Weights [N rows, K cols], nb = K/32 blocks per row:
//   Q4 : codes  uint32 [N][nb][4]   dword k of a block = bytes (2k, 2k+1, 2k+8,
//                                   2k+9) of the reference's 16 packed bytes, i.e.
//                                   high nibbles = elements {2k,2k+1,2k+8,2k+9},
//                                   low nibbles = those + 16: the lane-k element
//                                   set of the reference's _mm_madd_epi16 dot
//        deltas uint16 [N][nb]
//   Q8 : codes  uint32 [N][nb][8]   dwords (2k, 2k+1) = elements {2k,2k+1,2k+8,2k+9}
//                                   and {2k+16,2k+17,2k+24,2k+25}
//        deltas uint16 [N][nb]
//   F16: uint16 [K/64][Npad][8][8]  for 64-column group g, row r, lane j: the 8
//                                   values at columns 64g + 8m + j (m = 0..7),
//                                   Npad = N rounded up to 8
#pragma once

#include <stddef.h>
#include <stdint.h>

#if defined(__HIPCC__)
#define NC_HD __host__ __device__ __forceinline__
#else
#define NC_HD inline
#endif

namespace nc {

enum Dtype : int { I32 = 0, F16 = 1, F32 = 2, Q8 = 3, Q4 = 4 };

NC_HD int qblocks(int cols) { return (cols + 31) / 32; }
NC_HD int round16(int b) { return (b + 15) & ~15; }

// Bytes of one activation row of `cols` values in dtype `dt`.
NC_HD int act_pitch(int dt, int cols)
{
    if (dt == Q8) return round16(qblocks(cols) * 34);
    if (dt == F16) return round16(cols * 2);
    return round16(cols * 4);
}

// Offset of the fp16 delta array inside a Q8 activation row.
NC_HD int act_delta_offset(int cols) { return qblocks(cols) * 32; }

}  // namespace nc
