// Internal helpers shared by the HIP translation units of liborc_hip.so.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#include "../../include/orc.h"

namespace orc {

// Error plumbing: the C ABI returns codes; the message is kept per thread.
int set_error(int code, const std::string& msg);
hipStream_t resolve_stream(orc_stream_t s);
bool initialized();
// Per-device GEMM state (CU count, LDS limit, split-K workspace), set up by orc_init.
int gemm_device_init(int device);
void gemm_device_release();
// Looks up this device's copy of orc_argmax_noalloc's scratch array (the
// device must be current); once per device, from orc_init.
int argmax_noalloc_device_init(int device);

// Live kernel timing (orc_prof_*): when enabled and the stream is not being
// captured, hands out a start / stop event pair for one launch and records
// it under (family, n_tok) with the launch's algorithmic bytes; returns false
// (events untouched) otherwise. Families: the GGML weight type of a GEMM, or
// one of the attention ids below.
constexpr int kProfAttnWG = ORC_PROF_ATTN_WG, kProfAttnSplit = ORC_PROF_ATTN_SPLIT, kProfAttnMerge = ORC_PROF_ATTN_MERGE,
              kProfAttnMt = ORC_PROF_ATTN_MT, kProfAttnPf = ORC_PROF_ATTN_PF;
bool prof_arm(hipStream_t s, int family, int n_tok, double bytes, hipEvent_t* start, hipEvent_t* stop);

#define ORC_HIP_CHECK(expr)                                                                       \
    do {                                                                                          \
        hipError_t e_ = (expr);                                                                   \
        if (e_ != hipSuccess)                                                                     \
            return ::orc::set_error(ORC_E_HIP, std::string(#expr) + ": " + hipGetErrorString(e_)); \
    } while (0)

#define ORC_LAUNCH_CHECK() ORC_HIP_CHECK(hipGetLastError())

// ── device helpers ───────────────────────────────────────────────────────────
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Exact IEEE half -> float (the hardware conversion is exact for all inputs,
// including subnormals, as the reference's fp16() is).
__device__ __forceinline__ float h2f(uint32_t bits16) {
    _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)bits16);
    return (float)h;
}

// Unaligned loads: gfx950 under HSA runs in unaligned-access mode, so these
// compile to single global_load_dword{,x2,x4} at any byte alignment.
typedef u32x4 __attribute__((aligned(1))) u32x4_u;
typedef u32x2 __attribute__((aligned(1))) u32x2_u;
typedef uint32_t __attribute__((aligned(1))) u32_u;
typedef uint16_t __attribute__((aligned(1))) u16_u;
__device__ __forceinline__ u32x4 ld16(const uint8_t* p) { return *(const u32x4_u*)p; }
__device__ __forceinline__ u32x2 ld8(const uint8_t* p) { return *(const u32x2_u*)p; }
__device__ __forceinline__ uint32_t ld4(const uint8_t* p) { return *(const u32_u*)p; }
__device__ __forceinline__ uint32_t ld2(const uint8_t* p) { return *(const u16_u*)p; }

// Byte k of w as float; the compiler emits one v_cvt_f32_ubyte{k}.
__device__ __forceinline__ float ubyte_f(uint32_t w, int k) { return (float)((w >> (8 * k)) & 0xFFu); }

// DPP lane exchange inside a row of 16 lanes, and the sum over each group of
// four consecutive lanes in a fixed order (xor 1, then xor 2)
template <int CTRL> __device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ float quad_sum(float v) {
    v += dpp<0xB1>(v);  // quad_perm [1,0,3,2]
    v += dpp<0x4E>(v);  // quad_perm [2,3,0,1]
    return v;
}

// Q4_K 6-bit (scale, min) of sub-block `is` from the 12 scale bytes held in
// three dwords (core/gguf_parser.cpp:1085-1093).
__device__ __forceinline__ void q4k_scale_min(int is, uint32_t s0, uint32_t s1, uint32_t s2, uint32_t& sc,
                                              uint32_t& mn) {
    if (is < 4) {
        sc = (s0 >> (8 * is)) & 63u;
        mn = (s1 >> (8 * is)) & 63u;
    } else {
        const int k = 8 * (is - 4);
        const uint32_t b8 = (s2 >> k) & 0xFFu;
        sc = (b8 & 0xFu) | (((s0 >> k) & 0xFFu) >> 6 << 4);
        mn = (b8 >> 4) | (((s1 >> k) & 0xFFu) >> 6 << 4);
    }
}

}  // namespace orc
