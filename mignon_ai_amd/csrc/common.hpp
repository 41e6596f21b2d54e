// Device helpers shared by the gfx950 kernels.
//
// Numerics follow the reference INT8 engine (W8A32: int8 weights with one fp32 scale per tensor, fp32
// activations). Everything here is built with -ffp-contract=off, so a*b+c rounds twice unless fmaf is
// written, exactly like the reference's Go code (which has no implicit FMA on amd64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mg {

typedef int v4i __attribute__((ext_vector_type(4)));

// A load through the global address space. Pointers read from device memory (the per-block weight
// tables of the one-workgroup decode steps) are generic, and generic (flat) loads count against both
// the memory and the LDS counters, so the compiler waits for every outstanding load and LDS access at
// each use: one fragment in flight instead of a batch.
template <class T>
__device__ __forceinline__ T ldg(const T* p) {
    return *(const __attribute__((address_space(1))) T*)p;
}
template <class T>
__device__ __forceinline__ void stg(T* p, T v) {
    *(__attribute__((address_space(1))) T*)p = v;
}
// float4 is a class type: through the native vector type
typedef float v4f_ __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ldg(const float4* p) {
    const v4f_ v = *(const __attribute__((address_space(1))) v4f_*)p;
    return float4{v.x, v.y, v.z, v.w};
}
__device__ __forceinline__ void stg(float4* p, float4 v) {
    *(__attribute__((address_space(1))) v4f_*)p = v4f_{v.x, v.y, v.z, v.w};
}

constexpr int WAVE = 64;

// Limb expansion of fp32 activations for int8 MFMA. A row segment x with scale s = amax/127 is held as
// three int8 digits q0, q1, q2 in [-127, 127] with x ~= s*(q0 + q1/254 + q2/254^2); each digit plane is
// multiplied by the int8 weights with exact int32 accumulation and the three sums are combined in fp32.
// Representation error is at most s*(0.5/64516 + 2^-23*127), about 1.2e-7*amax.
constexpr float kLimbBase = 254.0f;
constexpr float kInvLimb1 = 1.0f / 254.0f;
constexpr float kInvLimb2 = 1.0f / 64516.0f;
// Chunks whose largest magnitude is below this are stored as zero (127/amax would overflow).
constexpr float kTinyAmax = 1e-30f;

struct Limbs {
    int8_t q0, q1, q2;
};

__device__ __forceinline__ float clamp127(float v) { return fminf(fmaxf(v, -127.0f), 127.0f); }

// inv = 127/amax (0 when the chunk is zero). Integer-valued inputs with amax = 127 give inv = 1, so
// their first digit is the input itself and the other two are zero.
__device__ __forceinline__ Limbs split_limbs(float x, float inv) {
    float y = x * inv;
    float q0 = clamp127(rintf(y));
    float y1 = (y - q0) * kLimbBase;
    float q1 = clamp127(rintf(y1));
    float y2 = (y1 - q1) * kLimbBase;
    float q2 = clamp127(rintf(y2));
    return Limbs{(int8_t)q0, (int8_t)q1, (int8_t)q2};
}

// The three digits of four consecutive elements packed as three dwords (element e in byte e of each),
// equal to split_limbs' digits. Adding 1.5*2^23 rounds a value in [-2^22, 2^22] to the nearest integer
// (ties to even, like rintf) and leaves that integer's two's-complement low byte as the sum's low
// mantissa byte, so no clamp or float-to-int conversion is needed: |x*inv| <= 127 (up to rounding) by
// the choice of scale, and every residual times 254 lies in [-127, 127].
//
// Each residual (y - q)*254 is formed as fma(y, 254, fma(t, -254, 254*C)) with t = y + C: the inner fma is
// -254*q exactly (an integer of at most 32258), and the outer one rounds the exact 254*(y - q) once, which
// is what the product of the exact difference y - q and 254 rounds to. Eight operations per element.
__device__ __forceinline__ void digits3(float y, uint32_t& b0, uint32_t& b1, uint32_t& b2) {
    const float C = 12582912.0f;        // 1.5 * 2^23
    const float C254 = 254.0f * C;      // exact: 381 * 2^23
    const float t0 = y + C;
    const float y1 = fmaf(y, kLimbBase, fmaf(t0, -kLimbBase, C254));
    const float t1 = y1 + C;
    const float y2 = fmaf(y1, kLimbBase, fmaf(t1, -kLimbBase, C254));
    const float t2 = y2 + C;
    b0 = __float_as_uint(t0);
    b1 = __float_as_uint(t1);
    b2 = __float_as_uint(t2);
}

__device__ __forceinline__ void split4_pack(float4 x, float inv, uint32_t& w0, uint32_t& w1, uint32_t& w2) {
    const float xs[4] = {x.x, x.y, x.z, x.w};
    uint32_t b0[4], b1[4], b2[4];
#pragma unroll
    for (int e = 0; e < 4; e++) digits3(xs[e] * inv, b0[e], b1[e], b2[e]);
    // v_perm_b32: selector bytes 0-3 take the second operand's bytes, 4-7 the first's, 0x0c gives zero
    w0 = __builtin_amdgcn_perm(b0[1], b0[0], 0x0c0c0400u) | __builtin_amdgcn_perm(b0[3], b0[2], 0x04000c0cu);
    w1 = __builtin_amdgcn_perm(b1[1], b1[0], 0x0c0c0400u) | __builtin_amdgcn_perm(b1[3], b1[2], 0x04000c0cu);
    w2 = __builtin_amdgcn_perm(b2[1], b2[0], 0x0c0c0400u) | __builtin_amdgcn_perm(b2[3], b2[2], 0x04000c0cu);
}

// split4_pack for two consecutive elements: their digits in bytes 0 and 1 of each word.
__device__ __forceinline__ void split2_pack(float2 x, float inv, uint32_t& w0, uint32_t& w1, uint32_t& w2) {
    const float xs[2] = {x.x, x.y};
    uint32_t b0[2], b1[2], b2[2];
#pragma unroll
    for (int e = 0; e < 2; e++) digits3(xs[e] * inv, b0[e], b1[e], b2[e]);
    w0 = __builtin_amdgcn_perm(b0[1], b0[0], 0x0c0c0400u);
    w1 = __builtin_amdgcn_perm(b1[1], b1[0], 0x0c0c0400u);
    w2 = __builtin_amdgcn_perm(b2[1], b2[0], 0x0c0c0400u);
}

// Base-256 digits of four consecutive elements for the GEMMs that read an fp32 operand (launch_gemm_fa).
// With inv about 2^22/amax (limb256_scale), fma(x, inv, 1.5*2^23) rounds x*inv to the nearest integer q
// (ties to even; |q| < 2^22) and its bit pattern is 0x4B400000 + q. The signed-byte digits of
// q = 65536*q0 + 256*q1 + q2 are q2 = the low byte of q, q1 = byte 1 of q + 0x80 and q0 = byte 2 of
// q + 0x8080 (so |q0| <= 64). With z = that pattern + 0x8080 - 0x400000 (byte 3 aside, q + 0x8080), q0 is
// byte 2 of z, and bytes 1 and 0 of z are q1 and q2 with bit 7 flipped (adding 0x8000 flips bit 15 and
// leaves bits 0-14; adding 0x80 to a byte flips its bit 7). w0 holds q0 of the four elements (element e in
// byte e), w1 q1, w2 q2. Seventeen operations for the four elements.
__device__ __forceinline__ void digits256_4(float4 x, float inv, uint32_t& w0, uint32_t& w1, uint32_t& w2) {
    const float C = 12582912.0f;  // 1.5 * 2^23
    const uint32_t z0 = __float_as_uint(fmaf(x.x, inv, C)) - 0x3F7F80u, z1 = __float_as_uint(fmaf(x.y, inv, C)) - 0x3F7F80u,
                   z2 = __float_as_uint(fmaf(x.z, inv, C)) - 0x3F7F80u, z3 = __float_as_uint(fmaf(x.w, inv, C)) - 0x3F7F80u;
    // v_perm_b32: selector bytes 0-3 take the second operand's bytes, 4-7 the first's, 0x0c gives zero
    const uint32_t a01 = __builtin_amdgcn_perm(z1, z0, 0x05010400u);  // bytes 0 of z0, z1, bytes 1 of z0, z1
    const uint32_t a23 = __builtin_amdgcn_perm(z3, z2, 0x05010400u);
    w2 = __builtin_amdgcn_perm(a23, a01, 0x05040100u) ^ 0x80808080u;
    w1 = __builtin_amdgcn_perm(a23, a01, 0x07060302u) ^ 0x80808080u;
    w0 = __builtin_amdgcn_perm(z1, z0, 0x0c0c0602u) | __builtin_amdgcn_perm(z3, z2, 0x06020c0cu);
}
// inv of digits256_4 for a row whose largest magnitude is amax (0 for a zero row): (2^22 - 256)/amax, so
// that |x*inv| stays below 2^22 whatever the roundings; and the row's scale 65536/inv (about amax/64) by
// which the combined digit sums q0 + q1/256 + q2/65536 are multiplied.
__device__ __forceinline__ void limb256_scale(float amax, float& scale, float& inv) {
    if (amax < kTinyAmax) {
        scale = 0.0f;
        inv = 0.0f;
    } else {
        inv = 4194048.0f / amax;
        scale = 65536.0f / inv;
    }
}
// The three digit-plane sums (p0, p1, p2) of a dot product over K <= 512 combined as p0 + (254 p1 + p2)/254^2
// with the two lower planes joined exactly in integers first: |p1|, |p2| <= 127*127*512 < 2^23, so one
// v_mad_i32_i24 forms 254 p1 + p2 (< 2^31 in magnitude), and the sum costs four instructions instead of five.
// The result differs from the three-term form by the rounding of the two conversions only.
__device__ __forceinline__ float limb_sum_k512(int p0, int p1, int p2) {
    return fmaf((float)(__mul24(p1, 254) + p2), 1.0f / 64516.0f, (float)p0);
}
constexpr float kInvLimb256_1 = 1.0f / 256.0f;
constexpr float kInvLimb256_2 = 1.0f / 65536.0f;

__device__ __forceinline__ void limb_scale(float amax, float& scale, float& inv) {
    if (amax < kTinyAmax) {
        scale = 0.0f;
        inv = 0.0f;
    } else {
        scale = amax / 127.0f;
        inv = 127.0f / amax;
    }
}

// quant.sigmoidClamped (internal/quant/stream.go:127-136): 1/(1 + float32(exp(float64(-x)))),
// saturated beyond |x| > 15.
__device__ __forceinline__ float sigmoid_clamped(float x) {
    if (x > 15.0f) return 1.0f;
    if (x < -15.0f) return 0.0f;
    return 1.0f / (1.0f + (float)exp((double)(-x)));
}

// sigmoidClamped evaluated with the hardware exponential and reciprocal (v_exp_f32, v_rcp_f32): used in
// GEMM epilogues, where the reference's float64 exp and a correctly rounded division per output would
// cost as much VALU time as the matrix work. For |x| <= 15 the relative error is below 2e-6 (the
// argument rounding of x*log2(e) dominates), far inside the engine's 1e-4 output tolerance.
__device__ __forceinline__ float sigmoid_clamped_f32(float x) {
    if (x > 15.0f) return 1.0f;
    if (x < -15.0f) return 0.0f;
    return __builtin_amdgcn_rcpf(1.0f + __expf(-x));
}

// sigmoidClamped from 2^x and the hardware reciprocal (see sigmoid_clamped_f32), as the GEMM epilogues
// compute it; exactly 0 and 1 beyond |x| > 15 as in the reference.
// The empty volatile asm pins the exponential and reciprocal before the saturation test: otherwise the
// compiler moves them into a branch of their own, one divergent branch per element.
__device__ __forceinline__ float sigmoid_epi(float x) {
    const float e = __builtin_amdgcn_exp2f(x * -1.4426950408889634f);
    float v = __builtin_amdgcn_rcpf(1.0f + e);
    asm volatile("" : "+v"(v));
    const float sat = x > 0.0f ? 1.0f : 0.0f;
    return fabsf(x) > 15.0f ? sat : v;
}

// One element of the reference's vectorised e^x (vecExpASM_F32, internal/kernels/vec_amd64.s:281-430):
// clamp to [-88, 88], k = nearest-even(x*log2e), two-constant ln2 reduction with FMA, degree-5
// polynomial as an FMA chain, 2^k from exponent bits. Bit-identical to the reference on IEEE FMA.
__device__ __forceinline__ float fast_exp_ref(float x) {
    const float invLn2 = __uint_as_float(0x3fb8aa3bu), ln2Hi = __uint_as_float(0x3f317200u),
                ln2Lo = __uint_as_float(0x35bfbe8eu);
    const float c2 = 0.5f, c3 = __uint_as_float(0x3e2aaaabu), c4 = __uint_as_float(0x3d2aaaabu),
                c5 = __uint_as_float(0x3c088889u);
    x = (x < 88.0f) ? x : 88.0f;
    x = (x > -88.0f) ? x : -88.0f;
    float k = rintf(x * invLn2);
    float r = fmaf(-k, ln2Hi, x);
    r = fmaf(-k, ln2Lo, r);
    float p = fmaf(r, c5, c4);
    p = fmaf(r, p, c3);
    p = fmaf(r, p, c2);
    p = fmaf(r, p, 1.0f);
    p = fmaf(r, p, 1.0f);
    int ki = (int)k + 127;
    return p * __uint_as_float((uint32_t)ki << 23);
}

// Horizontal reduction of the reference's 8-lane AVX2 accumulators (vec_amd64.s:38-44): lanes i and
// i+4, then pairs (0,2), (1,3), then the two results.
__device__ __forceinline__ float hreduce8(const float v[8]) {
    float f0 = v[0] + v[4], f1 = v[1] + v[5], f2 = v[2] + v[6], f3 = v[3] + v[7];
    float g0 = f0 + f2, g1 = f1 + f3;
    return g0 + g1;
}

// kernels.DotF32 as dotProductASM_F32 computes it (internal/kernels/vec_amd64.s:4-63), sequentially in
// one lane: two 8-lane FMA accumulators over 16-chunks, an 8-chunk into the first, the tree, then the
// unfused scalar tail. x may live in registers (compile-time indexing after unrolling), y anywhere.
template <int N, class X, class Y>
__device__ __forceinline__ float dot_f32_ref(const X& x, const Y& y) {
    float a0[8], a1[8];
#pragma unroll
    for (int j = 0; j < 8; j++) { a0[j] = 0.0f; a1[j] = 0.0f; }
    int i = 0;
#pragma unroll
    for (; i + 16 <= N; i += 16) {
#pragma unroll
        for (int j = 0; j < 8; j++) {
            a0[j] = fmaf(x[i + j], y[i + j], a0[j]);
            a1[j] = fmaf(x[i + 8 + j], y[i + 8 + j], a1[j]);
        }
    }
    if (i + 8 <= N) {
#pragma unroll
        for (int j = 0; j < 8; j++) a0[j] = fmaf(x[i + j], y[i + j], a0[j]);
        i += 8;
    }
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; j++) v[j] = a0[j] + a1[j];
    float s = hreduce8(v);
#pragma unroll
    for (; i < N; i++) {
        float p = x[i] * y[i];
        s = s + p;
    }
    return s;
}

// Lane-exchange move within rows of 16 lanes (DPP: a VALU operand modifier, no LDS round trip).
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_value(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Maximum over the 64 lanes (all active), returned to every lane: within each row of 16 by DPP (swap
// neighbours, swap pairs, half-row mirror, row mirror), then the four rows' values read out. The maximum
// does not depend on the order of the comparisons.
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_move<0xB1>(v));   // quad_perm [1, 0, 3, 2]
    v = fmaxf(v, dpp_move<0x4E>(v));   // quad_perm [2, 3, 0, 1]
    v = fmaxf(v, dpp_move<0x141>(v));  // row_half_mirror
    v = fmaxf(v, dpp_move<0x140>(v));  // row_mirror
    return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)), fmaxf(lane_value(v, 32), lane_value(v, 48)));
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__host__ __device__ constexpr int round_up(int a, int b) { return (a + b - 1) / b * b; }

// Grid mapping that keeps consecutive tiles on one XCD: the dispatcher places workgroup b on XCD b % 8,
// so tile t goes to XCD t / per_xcd. Tiles sharing an activation row block are consecutive, which makes
// the weight sweep over one row block hit the same XCD's L2.
__device__ __forceinline__ int xcd_tile(int b, int total) {
    int per = (total + 7) / 8;
    return (b % 8) * per + b / 8;
}
__host__ __forceinline__ int xcd_grid(int total) { return 8 * ((total + 7) / 8); }

}  // namespace mg
