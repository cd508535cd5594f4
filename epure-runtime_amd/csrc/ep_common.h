// Shared device helpers for the gfx950 kernels: element conversions, the
// per-row power-of-two activation rescale, and wave reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "epure_hip.h"

typedef _Float16 f16_t;
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

#define EP_DEV __device__ __forceinline__

EP_DEV float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// float -> bfloat16, round to nearest even (NaN stays NaN).
EP_DEV uint16_t f32_to_bf16(float f)
{
    const uint32_t u = __float_as_uint(f);
    const uint32_t rounded = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
    const uint32_t nan = (u >> 16) | 0x40u;
    return (uint16_t)((u & 0x7fffffffu) > 0x7f800000u ? nan : rounded);  // a select, no branch
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Bit reinterpretations go through memcpy: __builtin_bit_cast of an
// ext-vector element to a 16-bit-lane vector is lowered to element 0 by this
// compiler (every lane of a u32x4 read as lane 0).
EP_DEV uint16_t f16_bits(f16_t h)
{
    uint16_t u;
    __builtin_memcpy(&u, &h, 2);
    return u;
}
EP_DEV f16_t f16_from_bits(uint16_t b)
{
    f16_t h;
    __builtin_memcpy(&h, &b, 2);
    return h;
}
EP_DEV f16x2_t as_f16x2(uint32_t u)
{
    f16x2_t v;
    __builtin_memcpy(&v, &u, 4);
    return v;
}
EP_DEV bf16x2_t as_bf16x2(uint32_t u)
{
    bf16x2_t v;
    __builtin_memcpy(&v, &u, 4);
    return v;
}

// Load element i of a buffer of element type `dt` as float.
EP_DEV float load_as_f32(const void *p, int dt, int64_t i)
{
    if (dt == EP_F32)
        return ((const float *)p)[i];
    if (dt == EP_F16)
        return (float)((const f16_t *)p)[i];
    return bf16_to_f32(((const uint16_t *)p)[i]);
}

EP_DEV void store_from_f32(void *p, int dt, int64_t i, float v)
{
    if (dt == EP_F32)
        ((float *)p)[i] = v;
    else if (dt == EP_F16)
        ((f16_t *)p)[i] = (f16_t)v;
    else
        ((uint16_t *)p)[i] = f32_to_bf16(v);
}

// Exponent e such that 2^13 <= amax * 2^-e < 2^14 for the largest |x| of a
// row (amax): every element converts to fp16 without overflow and rows of
// tiny values are lifted into the normal fp16 range.  2^-e and 2^e are
// exact (e is clamped to [-110, 110], inside float32's normal range), so
// rescaling changes no bf16 value and the result is scaled back exactly.
// Returns 0 for amax == 0 or non-finite.
EP_DEV int row_exponent(float amax)
{
    if (!(amax > 0.0f) || amax > 3.0e38f)
        return 0;
    int e;
    frexpf(amax, &e);      // amax = f * 2^e, f in [0.5, 1)  ->  amax < 2^e
    int s = e - 14;        // amax * 2^-s < 2^14
    if (s < -110)
        s = -110;
    if (s > 110)
        s = 110;
    return s;
}

// Workgroup barrier ordering LDS only: waits for this wave's LDS (and
// scalar) operations, then s_barrier.  __syncthreads() also waits for every
// global load and store of the wave still in flight (vmcnt), which would
// serialize a prologue with the weight loads it is meant to overlap.
EP_DEV void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Raw buffer descriptor over `bytes` bytes at a wave-uniform base p: a load
// at an offset past the end reads zeros.  Base and size go through
// readfirstlane so the descriptor is known to live in scalar registers (one
// the compiler cannot prove uniform turns every load into a per-lane
// waterfall loop).
EP_DEV __amdgpu_buffer_rsrc_t buffer_rsrc(const void *p, uint32_t bytes = 0x7fffffffu)
{
    const uint64_t v = (uint64_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return __builtin_amdgcn_make_buffer_rsrc((void *)(((uint64_t)hi << 32) | lo), 0,
                                             (int)__builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}

// Cross-workgroup hand-off without device-scope fences.  On gfx950 a
// device-scope fence writes back and invalidates the whole L2 of the XCD;
// instead, values another workgroup will read are stored and loaded as
// relaxed agent-scope atomics (coherent sc1 accesses), and the writer waits
// for its stores to complete before it bumps the hand-off counter.
template <typename T>
EP_DEV void st_agent(T *p, T v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
EP_DEV T ld_agent(T *p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
EP_DEV void wait_stores() { __builtin_amdgcn_s_waitcnt(0); }
EP_DEV int counter_add(int *p, int v)
{
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Cross-lane reductions without the LDS unit (a ds_bpermute round trip
// costs ~100 cycles, and a butterfly chains six of them): DPP within 16-lane
// rows (row_ror 8, row_ror 4, quad_perm [2,3,0,1], quad_perm [1,0,3,2]),
// then lanes l ^ 16 and l ^ 32 through v_permlane16/32_swap (gfx950).
// Every lane ends with the same value (each step pairs commutatively).
// All 64 lanes must be active.
template <int CTRL>
EP_DEV float dpp_mov(float v)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
EP_DEV float xor16_sum(float v)
{
    const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}
EP_DEV float xor32_sum(float v)
{
    const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}
EP_DEV float xor16_max(float v)
{
    const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}
EP_DEV float xor32_max(float v)
{
    const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}

// Butterfly sums over the 64 lanes through ds_bpermute (the per-layer
// kernels' order of additions).
EP_DEV float wave_sum_bfly(float v)
{
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1)
        v += __shfl_xor(v, o, 64);
    return v;
}
EP_DEV float wave_max_bfly(float v)
{
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1)
        v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Sum over the 64 lanes of a wave (result valid in every lane).
EP_DEV float wave_sum(float v)
{
    v += dpp_mov<0x128>(v);
    v += dpp_mov<0x124>(v);
    v += dpp_mov<0x4e>(v);
    v += dpp_mov<0xb1>(v);
    return xor32_sum(xor16_sum(v));
}

EP_DEV float wave_max(float v)
{
    v = fmaxf(v, dpp_mov<0x128>(v));
    v = fmaxf(v, dpp_mov<0x124>(v));
    v = fmaxf(v, dpp_mov<0x4e>(v));
    v = fmaxf(v, dpp_mov<0xb1>(v));
    return xor32_max(xor16_max(v));
}
