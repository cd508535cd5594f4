// Device building blocks of the LUT dequant-GEMV, shared by the per-linear
// kernels (gemv.hip) and the persistent decode step (step.hip).
//
// Dequantization is an LDS "pair table": byte value b -> half2(cb[b & 15],
// cb[b >> 4]) for 4-bit indices (low nibble = even k, epure/runtime.py:45),
// or the single fp16 cb[b] duplicated for 8-bit indices.  Entry b holds 32
// copies at bytes (b << 8) + 4 c (the upper half of each 256-byte entry is
// unused) and lane l reads copy l & 31, so a ds_read_b32 with random byte
// values never has two lanes of one 32-lane half on one bank.  The byte
// address of a lookup is (b << 8) | ((lane & 31) << 2), formed by one
// v_perm from the packed word.
#pragma once

#include "ep_common.h"

namespace ep {

constexpr int kTabDwords = 256 * 64;     // 64 KiB per table (32 copies per 256-byte entry used)
constexpr int kTabBytes = kTabDwords * 4;
constexpr int kTabCopies = 32;
constexpr int kSlabBytes = 256;          // bytes of a row covered by 16 lanes x 16 B

// Fills one pair table from the codebook's fp16 bits (cb16[l] = 0 for
// l >= levels, as the Rust LUT's zeros, kernel/src/lib.rs:58-59): 2048
// 16-byte stores per workgroup, the codebook reads of four at a time issued
// together.
template <int BITS>
EP_DEV void build_table(uint32_t *tab, const uint16_t *cb16)
{
#pragma unroll 4
    for (int i = threadIdx.x; i < 256 * kTabCopies / 4; i += blockDim.x) {
        const int b = i >> 3;  // entry; (i & 7) = its 16-byte piece
        uint32_t v;
        if constexpr (BITS == 4) {
            v = (uint32_t)cb16[b & 15] | ((uint32_t)cb16[b >> 4] << 16);
        } else {
            const uint32_t h = cb16[b];
            v = h | (h << 16);
        }
        ((u32x4_t *)tab)[b * 16 + (i & 7)] = (u32x4_t){v, v, v, v};
    }
}

// v_perm selectors building the LDS byte address (byte_i << 8) | lane4:
// result byte0 = lane4 (src1 byte 0), byte1 = byte i of the packed word
// (src0 byte i = selector 4 + i), bytes 2-3 = 0 (selector 12).
constexpr uint32_t kSelByte[4] = {0x0c0c0400u, 0x0c0c0500u, 0x0c0c0600u, 0x0c0c0700u};
// Two pair tables interleaved in 64 KiB (the one-launch step): entry b of
// table `slot`, copy c (of 32) at dword b * 64 + slot * 32 + c, i.e. byte
// (b << 8) | (slot << 7) | (c << 2) -- the kSelByte address with src1 =
// slot << 7 | (lane & 31) << 2.  32 copies serve a wave as fast as 64 (a
// ds_read_b32 takes 32 lanes per cycle).
constexpr int kPairTabBytes = 256 * 2 * 32 * 4;

EP_DEV uint32_t lds_read_u32(const uint32_t *base, uint32_t byte_addr)
{
    return *(const uint32_t *)((const char *)base + byte_addr);
}

template <int CTRL>
EP_DEV float dpp_f(float v)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Sum over the 16 lanes of a DPP row (lanes 16r..16r+15), in every lane:
// row_ror 8, row_ror 4, quad_perm [2,3,0,1], quad_perm [1,0,3,2].
EP_DEV float row16_sum(float v)
{
    v += dpp_f<0x128>(v);
    v += dpp_f<0x124>(v);
    v += dpp_f<0x4e>(v);
    v += dpp_f<0xb1>(v);
    return v;
}

// Two raw 16-bit activations (bf16 or fp16, per XDT) -> floats.
template <int XDT>
EP_DEV void unpack_pair(uint32_t raw, float &lo, float &hi)
{
    if constexpr (XDT == EP_BF16) {
        lo = __uint_as_float(raw << 16);
        hi = __uint_as_float(raw & 0xffff0000u);
    } else {
        lo = (float)f16_from_bits((uint16_t)(raw & 0xffffu));
        hi = (float)f16_from_bits((uint16_t)(raw >> 16));
    }
}

// silu(g) * u with the hardware reciprocal (about 1 ulp; the result is
// rounded to fp16 right after, so a correctly rounded divide buys nothing).
EP_DEV float silu_mul(float g, float u)
{
    return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
}

}  // namespace ep
