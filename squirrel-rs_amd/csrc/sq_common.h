// Shared definitions for the squirrel-hip library: status codes, device weight
// layouts and small device helpers used by every kernel file.
#pragma once
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

#include "../../include/squirrel_hip.h"

namespace sq {

// GGML type ids used on the path (src/file_parser/ggml_type.rs:8-41).
enum WType : int { WT_F32 = 0, WT_Q4_0 = 2, WT_Q8_0 = 8, WT_BF16 = 30 };

// Records a message for sq_last_error() and returns `code`.
int set_error(int code, const std::string& msg);

// The f32-activation matvec / matmul kernels (BF16 weights and the
// SQUIRREL_F32_ACTS ablation) are switched off: a BF16 model prefill hit a GPU
// memory fault whose cause is not yet identified.  Every entry point that
// would launch them returns SQ_ERR_UNSUPPORTED with this message.
constexpr const char* kA32Disabled =
    "f32-activation kernels (BF16 weights, SQUIRREL_F32_ACTS) are disabled pending analysis "
    "of a GPU fault";

#define SQ_HIP_CHECK(expr)                                                            \
    do {                                                                              \
        hipError_t e_ = (expr);                                                       \
        if (e_ != hipSuccess)                                                         \
            return ::sq::set_error(SQ_ERR_HIP, std::string(#expr) + ": " +            \
                                                   hipGetErrorString(e_));           \
    } while (0)

// A weight matrix resident in HBM, repacked from GGUF blocks at upload.
//
// GGUF stores a [k, rows] matrix as `rows` rows of k/32 blocks (34 B Q8_0,
// 18 B Q4_0, 64 B of bf16).  On the device the block payloads and the block
// scales are split so that every lane of a wavefront can fetch one whole
// block payload with aligned 16-byte loads:
//   Q8_0: qs  int8  [rows][k]        scale f16 [rows][k/32]
//   Q4_0: qs  uint8 [rows][k/2]      scale f16 [rows][k/32]
//         (each block's 16 bytes in GGUF order: low nibble = element j,
//          high nibble = element j+16, value (q-8)*scale)
//   BF16: qs  bf16  [rows][k]        scale unused
// Bytes per weight are unchanged (1.0625 / 0.5625 / 2).
struct DevMatrix {
    int wtype = 0;
    int rows = 0;
    int k = 0;
    void* qs = nullptr;
    uint16_t* scale = nullptr;
    size_t payload_bytes() const;
    size_t scale_bytes() const;
};

// Device-side views passed to kernels by value.
struct MatView {
    const void* qs;
    const uint16_t* scale;
    int rows;
    int k;
    int wtype;
    int pad = 0;  // the struct's tail, zero rather than whatever the stack held
};

inline MatView view(const DevMatrix& m) { return MatView{m.qs, m.scale, m.rows, m.k, m.wtype}; }

}  // namespace sq

// ---------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------
#if defined(__HIPCC__)

__device__ __forceinline__ float sq_f16_to_f32(uint16_t b) {
    return (float)__builtin_bit_cast(_Float16, b);
}

// IEEE binary16 conversion, round to nearest even (v_cvt_f16_f32 in the
// default rounding mode).
__device__ __forceinline__ uint16_t sq_f32_to_f16(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

__device__ __forceinline__ float sq_bf16_to_f32(uint16_t b) {
    return __builtin_bit_cast(float, (uint32_t)b << 16);
}

// Wavefront reductions through DPP row operations and lane reads, with no
// LDS traffic; every lane of the wavefront must be active, and every lane
// gets the result.  Quad swaps, the half-row and row mirrors leave each lane
// with its 16-lane row's value; row_bcast:15 / :31 then carry rows into the
// upper rows, and lanes 31 / 63 are read back.
template <int CTRL, int ROWS>
__device__ __forceinline__ float sq_dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROWS, 0xF, false));
}
// the same, with lanes outside ROWS keeping their own value
template <int CTRL, int ROWS>
__device__ __forceinline__ float sq_dpp_keep(float v) {
    const int b = __builtin_bit_cast(int, v);
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(b, b, CTRL, ROWS, 0xF, false));
}
__device__ __forceinline__ float sq_row_max(float v) {
    v = fmaxf(v, sq_dpp<0xB1, 0xF>(v));   // quad_perm [1,0,3,2]
    v = fmaxf(v, sq_dpp<0x4E, 0xF>(v));   // quad_perm [2,3,0,1]
    v = fmaxf(v, sq_dpp<0x141, 0xF>(v));  // row_half_mirror
    return fmaxf(v, sq_dpp<0x140, 0xF>(v));  // row_mirror
}

__device__ __forceinline__ float sq_wave_sum(float v) {
    v += sq_dpp<0xB1, 0xF>(v);
    v += sq_dpp<0x4E, 0xF>(v);
    v += sq_dpp<0x141, 0xF>(v);
    v += sq_dpp<0x140, 0xF>(v);
    v += sq_dpp<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
    v += sq_dpp<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3: lane 63 holds the sum
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

__device__ __forceinline__ float sq_wave_max(float v) {
    v = sq_row_max(v);
    v = fmaxf(v, sq_dpp_keep<0x142, 0xA>(v));
    v = fmaxf(v, sq_dpp_keep<0x143, 0xC>(v));
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Maximum within each aligned group of 32 lanes (one 32-element block).
__device__ __forceinline__ float sq_half_max(float v) {
    v = sq_row_max(v);
    v = fmaxf(v, sq_dpp_keep<0x142, 0xA>(v));  // lanes 31 and 63 hold the two halves' maxima
    const float lo = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 31));
    const float hi = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
    return (threadIdx.x & 32) ? hi : lo;
}

// Maximum over each lane quad (every lane of the wavefront active): the
// 32-element block of a thread that holds 8 consecutive elements.
__device__ __forceinline__ float sq_quad_max(float v) {
    v = fmaxf(v, sq_dpp<0xB1, 0xF>(v));  // quad_perm [1,0,3,2]
    return fmaxf(v, sq_dpp<0x4E, 0xF>(v));  // quad_perm [2,3,0,1]
}

// The Q8_0 activation quantizer of the reference, for one element whose block
// amax is known: quantize_row_q8_0_scalar (src/kernels/dot_prod.rs:21-31).
// scale = amax/127 (IEEE division), inv = scale > 0 ? 1/scale : 0,
// q = clamp(round_half_away(x*inv), -127, 127) with NaN -> 0.
__device__ __forceinline__ float sq_q8_scale(float amax) { return amax / 127.0f; }
__device__ __forceinline__ float sq_q8_inv(float scale) {
    return scale > 0.0f ? 1.0f / scale : 0.0f;
}
__device__ __forceinline__ int8_t sq_q8_quant(float x, float inv) {
    float v = roundf(x * inv);
    if (v < -127.0f) v = -127.0f;
    if (v > 127.0f) v = 127.0f;
    return (v != v) ? (int8_t)0 : (int8_t)(int)v;
}

// One block's contribution on the integer path, (f32(isum) * sa) * sw, with
// no fused multiply-add: dot_q8_0_q8_0_scalar (src/kernels/dot_prod.rs:385).
__device__ __forceinline__ float sq_q_term(int isum, float sa, float sw) {
#pragma clang fp contract(off)
    float t = (float)isum * sa;
    return t * sw;
}

// One RoPE pair rotation without contraction (src/kernels/rope.rs:28-31):
// (a, b) -> (a*c - b*s, a*s + b*c).
__device__ __forceinline__ void sq_rotate(float a, float b, float c, float s, float& o0,
                                          float& o1) {
#pragma clang fp contract(off)
    o0 = a * c - b * s;
    o1 = a * s + b * c;
}

// Sign-extended byte k (0..3) of a packed dword, as f32.
__device__ __forceinline__ float sq_sbyte_f(int dw, int k) {
    return (float)((int)((unsigned)dw << (24 - 8 * k)) >> 24);
}

typedef int sq_v4i __attribute__((ext_vector_type(4)));

// sigmoid_f32 (src/kernels/sigmoid.rs:2-9) and silu_f32 (silu.rs:4-8):
// x >= 0 ? 1 / (1 + exp(-x)) : exp(x) / (1 + exp(x)).  Both branches take
// exp of -|x| (the same argument, so the same bits), formed once here; as
// written with two branches the compiler evaluated both exponentials.
__device__ __forceinline__ float sq_sigmoid(float x) {
    const float e = expf(-fabsf(x));
    return (x >= 0.0f ? 1.0f : e) / (1.0f + e);
}

#endif  // __HIPCC__
