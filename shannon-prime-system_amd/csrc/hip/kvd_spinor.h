// kvd_spinor.h -- the Spinor-63 KV codec of SP_KV_SPINOR / SP_KV_SPINOR_REF
// sessions on the device.
//
// Reference semantics (core/vht2/vht2.c:59-104, spinor_block.c:59-149,
// core/session/sp_session.c:298-323):  a stored K or V head of HD coordinates
// is split into nb = ceil(HD/55) contiguous chunks of HD/nb coordinates, the
// first HD % nb one longer; each chunk keeps scale = max|v| (0 -> 1) and the
// int8 codes c = clamp(round_half_away((v / scale) * 127), +-127); attention
// reads v' = (float)c * (scale / 127).  The reference's 63-byte block adds a
// fixed header, a Mobius order of the 55 body bytes and a CRC-8; none of them
// changes v', so the device keeps the codes in coordinate order and the
// chunk multipliers beside them:
//
//   row = [HD int8 codes][nb float32 multipliers scale/127][zero pad to 16 B]
//
// Float mode stores these rows (K part then V part of a page, like the f32
// rows they replace); exact mode stores the usual int32 grid values of v'.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kvd {

constexpr int SPN_BODY = 55;                       // coordinates per block
enum KvCodec { KVC_PLAIN = 0, KVC_SPINOR = 1 };

__host__ __device__ constexpr int spn_blocks(int hd) { return hd <= SPN_BODY ? 1 : (hd + SPN_BODY - 1) / SPN_BODY; }
__host__ __device__ constexpr int spn_row_bytes(int hd) { return (hd + 4 * spn_blocks(hd) + 15) / 16 * 16; }
// chunk of coordinate e (the balanced split)
__host__ __device__ constexpr int spn_block_of(int hd, int e) {
    const int nb = spn_blocks(hd), base = hd / nb, big = (hd % nb) * (base + 1);
    return e < big ? e / (base + 1) : hd % nb + (e - big) / base;
}
// first coordinate of chunk b (b <= nb: nb gives hd)
__host__ __device__ constexpr int spn_block_start(int hd, int b) {
    const int nb = spn_blocks(hd), base = hd / nb, extra = hd % nb;
    return b * base + (b < extra ? b : extra);
}

// the int8 code of v in a chunk of the given scale: (v / scale) * 127 in float,
// then round half away from zero as floor(x + 0.5) / ceil(x - 0.5) in float
__device__ __forceinline__ int32_t spn_code(float v, float scale) {
    const float x = (v / scale) * 127.0f;
    const float r = x >= 0.0f ? floorf(x + 0.5f) : ceilf(x - 0.5f);
    const float c = fminf(fmaxf(r, -127.0f), 127.0f);
    return (int32_t)c;
}
__device__ __forceinline__ float spn_scale(float amax) { return amax > 0.0f ? amax : 1.0f; }

}  // namespace kvd
