// lmx_lanes.hpp -- cross-lane exchange inside a 64-wide wavefront without
// the LDS (device code only; included by the .hip sources).
//
// lane_xor<D>(v, lane) returns the value of v held by lane (lane ^ D), for D a
// power of two below 64:
//   D = 1, 2   DPP quad_perm [1,0,3,2] / [2,3,0,1]
//   D = 4      DPP quad_perm [3,2,1,0] (lane ^ 3), then row_half_mirror
//              (lane ^ 7 inside each 8-lane half row): lane ^ 4
//   D = 8      DPP row_ror:8 inside each 16-lane row: lane ^ 8
//   D = 16     v_permlane16_swap (gfx950): with both operands = v, the first
//              result holds row r-1's values in odd rows, the second row
//              r+1's values in even rows
//   D = 32     v_permlane32_swap (gfx950): the same for the two 32-lane halves
// All are VALU operations, so wave reductions and the FWHT butterflies leave
// the LDS pipe to the table reads.  Every lane of the wave must be active.
// lane_sum / lane_max / wave_max_key combine with lane ^ d for d = D, D/2,
// ..., 1, in that order, so every lane of the group gets the same bits.
#ifndef LMX_LANES_HPP
#define LMX_LANES_HPP

#include <hip/hip_runtime.h>

#include <cstdint>

namespace lmx {

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), CTRL, 0xF, 0xF, true));
}

template <int D>
__device__ __forceinline__ uint32_t lane_xor_u32(uint32_t v, int lane) {
  static_assert(D == 1 || D == 2 || D == 4 || D == 8 || D == 16 || D == 32, "lane distance");
  if constexpr (D == 1) {
    return dpp_u32<0xB1>(v);
  } else if constexpr (D == 2) {
    return dpp_u32<0x4E>(v);
  } else if constexpr (D == 4) {
    return dpp_u32<0x141>(dpp_u32<0x1B>(v));
  } else if constexpr (D == 8) {
    return dpp_u32<0x128>(v);
  } else if constexpr (D == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return (lane & 16) ? r[0] : r[1];
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return (lane & 32) ? r[0] : r[1];
  }
}

// For D = 16 or 32: lo / hi = the values of v in the lower / upper lane of
// the pair (l, l ^ D) that holds this lane, in both lanes of the pair.
template <int D>
__device__ __forceinline__ void lane_pair(float v, float &lo, float &hi) {
  static_assert(D == 16 || D == 32, "permlane swap distance");
  const uint32_t u = __float_as_uint(v);
  if constexpr (D == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    lo = __uint_as_float(r[0]);
    hi = __uint_as_float(r[1]);
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    lo = __uint_as_float(r[0]);
    hi = __uint_as_float(r[1]);
  }
}

template <int D>
__device__ __forceinline__ float lane_xor(float v, int lane) {
  return __uint_as_float(lane_xor_u32<D>(__float_as_uint(v), lane));
}

// Butterfly sum over the lanes l ^ d, d = D, D/2, ..., 1: every lane of a
// group of 2D lanes ends with the same bits (x + y and y + x agree).
template <int D>
__device__ __forceinline__ float lane_sum(float v, int lane) {
  v += lane_xor<D>(v, lane);
  if constexpr (D > 1) return lane_sum<D / 2>(v, lane);
  else return v;
}

// Butterfly sum over the lanes that share lane % RW (RW a power of two):
// lane ^ d for d = 32, 16, ..., RW; every lane of such a set ends with the
// same bits.
template <int RW, int D = 32>
__device__ __forceinline__ float strided_sum(float v, int lane) {
  if constexpr (D >= RW && D >= 1) {
    v += lane_xor<D>(v, lane);
    return strided_sum<RW, D / 2>(v, lane);
  } else {
    return v;
  }
}

template <int D>
__device__ __forceinline__ float lane_max(float v, int lane) {
  v = fmaxf(v, lane_xor<D>(v, lane));
  if constexpr (D > 1) return lane_max<D / 2>(v, lane);
  else return v;
}

// Largest 64-bit key over the wave; every lane gets it.
template <int D = 32>
__device__ __forceinline__ unsigned long long wave_max_key(unsigned long long key, int lane) {
  const uint32_t lo = lane_xor_u32<D>(uint32_t(key), lane), hi = lane_xor_u32<D>(uint32_t(key >> 32), lane);
  const unsigned long long o = (static_cast<unsigned long long>(hi) << 32) | lo;
  key = o > key ? o : key;
  if constexpr (D > 1) return wave_max_key<D / 2>(key, lane);
  else return key;
}

}  // namespace lmx

#endif  // LMX_LANES_HPP
