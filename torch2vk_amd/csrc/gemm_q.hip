// Prefill GEMM with block-quantized weights on the gfx950 matrix cores.
//
//   C[M, N] = A[M, K] . deq(W[N, K])^T      A bf16 row-major, W GGUF Q8_0 or Q4_K rows
//
// Replaces the reference's prefill matmuls (M > 8 tokens):
//   LINEAR_NOBIAS_Q8_0_F32  (src/models/quantized_qwen3/shaders/linear_nobias_q8_0_f32.py:24-209)
//   LINEAR_NOBIAS_Q4_K_F32  (src/models/quantized_qwen3/shaders/linear_nobias_q4_k_f32.py:26-296)
//   LLAMA_MATMUL_Q4_K_F32_{M,L} (src/models/optimized_qwen3/shaders/llama_matmul_q4_k_f32.py:32-141)
// They dequantise a weight tile into shared memory and run 16x16x16 fp16
// cooperative-matrix products; here the tile is dequantised to bf16 in LDS
// and fed to v_mfma_f32_32x32x16_bf16 with fp32 accumulation.
//
// Tiling.  A 512-thread block (8 waves, 2 x 4) computes a 256 x 256 tile of C;
// each wave owns 128 x 64 = 4 x 2 MFMA tiles of 32 x 32 (128 accumulator
// registers).  K advances 64 at a time through two LDS stages: while the
// matrix cores work on one stage, the next stage's A rows and packed weight
// blocks are already in flight to registers, and are dequantised into the
// other stage before the block barrier.  LDS rows are padded to 72 bf16
// (144 B) so the 16-B operand reads of 16 consecutive rows hit 16 distinct
// 4-bank groups.
//
// Operand layout of v_mfma_f32_32x32x16_bf16 (checked on the device): lane l
// supplies row (l % 32) of A and column (l % 32) of B, 8 consecutive k each,
// k = 8 * (l / 32) + j; the 16 results of lane l are C[8(i/4) + 4(l/32) + i%4][l % 32].
//
// Tile order.  Blocks are dealt round-robin to the 8 XCDs; the tile index is
// remapped so that each XCD walks a contiguous run of tiles, grouped 8 tiles
// down M, so the A rows and weight rows a group shares stay in that XCD's L2.
#include "common.h"

#include <type_traits>

namespace t2h {

constexpr int GQ_THREADS = 512;
constexpr int GQ_BN = 256;
constexpr int GQ_BK = 64;
constexpr int GQ_LDS_ROW = GQ_BK + 8;  // bf16 elements per padded LDS row
// Stage kt + 1's LDS stores spread over stage kt's four 16-deep MFMA steps (A in the first two, the weight
// dequantisation in the third), so that the VALU work runs while the matrix cores are busy instead of
// after them.
#ifndef GQ_SPLIT_STORE
#define GQ_SPLIT_STORE 1
#endif
#ifndef GQ_GROUP_M_DEF
#define GQ_GROUP_M_DEF 8
#endif
constexpr int GQ_GROUP_M = GQ_GROUP_M_DEF;  // tiles per group down M (4 and 8 measured fastest)

// GQEPI_GATED_F32: the SwiGLU form's gate | up tile columns written as fp32 products (split-K partials).
enum GemmEpilogue { GQEPI_F32 = 0, GQEPI_BF16 = 1, GQEPI_RESID = 2, GQEPI_SWIGLU = 3, GQEPI_GATED_F32 = 4 };

enum GemmAct { GQACT_NONE = 0, GQACT_GELU = 1 };

struct GemmArgs {
    const uint16_t* a;     // bf16 [M, K]
    const uint8_t* w;      // packed rows [N, row_bytes]
    void* c;               // [M, N] fp32 or bf16
    const float* residual; // GQEPI_RESID: fp32 [M, N] (may alias c)
    const float* bias;     // fp32 [N] or null
    int act;               // GemmAct, applied after the bias and before the residual
    uint32_t m, n, k;
    uint32_t row_bytes;
    uint32_t w_blocks;     // quant blocks per weight row; K columns past them multiply zeros
    uint32_t tiles_m, tiles_n;
    const uint8_t* w_up;   // GQEPI_SWIGLU: up rows (w holds the gate rows)
    uint32_t n_ff;         // GQEPI_SWIGLU: features; n = 2 n_ff
    uint32_t split_stages; // split-K: 64-wide K stages per split (blockIdx.y), split s writing its fp32
                           // products to c + s m n; 0: the whole K range in one pass
};

// Packed row of B-tile row r (0..255) of the tile at n0.  Plain: weight row
// n0 + r.  Gated (SwiGLU): each wave's 64 columns are 32 gate rows then the 32
// up rows of the same features, so the epilogue finds g and u in one lane:
// feature n0/2 + 32 (r / 64) + r % 32, from gate when (r / 32) is even.
template <bool GATED>
__device__ __forceinline__ const uint8_t* gemm_w_row(const GemmArgs& a, uint32_t n0, uint32_t r) {
    if constexpr (GATED) {
        uint32_t f = n0 / 2 + (r >> 6) * 32 + (r & 31);
        f = f < a.n_ff ? f : a.n_ff - 1;
        return ((r >> 5) & 1 ? a.w_up : a.w) + (size_t)f * a.row_bytes;
    } else {
        uint32_t row = n0 + r;
        row = row < a.n ? row : a.n - 1;
        return a.w + (size_t)row * a.row_bytes;
    }
}

// GELU of the bias + GELU epilogues (gelu_as: erf by Abramowitz-Stegun 7.1.26, as the reference's GELU)
__device__ __forceinline__ float gelu_erf(float v) { return gelu_as(v); }

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

// ------------------------------------------------------ weight formats ----

// Q8_0: thread t of the block dequantises block (t & 1) of the stage for row t >> 1.
struct GemmQ80 {
    static constexpr int BLOCK_VALUES = 32;
    static constexpr int BLOCK_BYTES = 34;
    static constexpr int ALIGN = 2;
    // MFMA step after which the next stage's A is stored, at 128- and at 256-row tiles (measured)
    static constexpr int STORE_STEP = 2, STORE_STEP_256 = 2;
    struct Raw {
        uint4 q0, q1;
        uint32_t d;
        bool inside;  // false: a block past the row's end, dequantised as zeros
    };
    template <bool GATED>
    __device__ static __forceinline__ void load(const GemmArgs& a, uint32_t n0, uint32_t k0, Raw& r) {
        const uint32_t t = threadIdx.x;
        // a stage past the row's last block (K padded to the 64-wide stage) reads
        // the last block again with a zero scale
        const uint32_t blk = k0 / 32 + (t & 1);
        const bool inside = blk < a.w_blocks;
        const uint8_t* p = gemm_w_row<GATED>(a, n0, t >> 1) + (size_t)(inside ? blk : a.w_blocks - 1) * 34;
        r.d = load_u16(p);  // unconditional (p is always inside the row) and not
        r.inside = inside;  // selected here, so nothing waits on the load before its use
        r.q0 = load_u4_ua(p + 2);
        r.q1 = load_u4_ua(p + 18);
    }
    // the block's 32 values as bf16 pairs: d * q, rounded once
    __device__ static __forceinline__ void convert(const Raw& r, uint32_t (&o)[16]) {
        const float d = r.inside ? f16_bits_to_f32(r.d) : 0.0f;
        const uint32_t q[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const uint32_t w = q[c];
            const float v0 = d * (float)(int8_t)(w & 0xffu);
            const float v1 = d * (float)(int8_t)((w >> 8) & 0xffu);
            const float v2 = d * (float)(int8_t)((w >> 16) & 0xffu);
            const float v3 = d * (float)(int8_t)(w >> 24);
            o[2 * c] = pack_bf16x2(v0, v1);
            o[2 * c + 1] = pack_bf16x2(v2, v3);
        }
    }
    // 32 bf16 values of this thread's block -> LDS row (t >> 1), columns 32 * (t & 1) ...
    __device__ static __forceinline__ void store(const Raw& r, uint16_t* lds_b) {
        const uint32_t t = threadIdx.x;
        uint32_t o[16];
        convert(r, o);
        uint16_t* dst = lds_b + (t >> 1) * GQ_LDS_ROW + (t & 1) * 32;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            *reinterpret_cast<uint4*>(dst + 8 * i) = make_uint4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
    }
};

// Q4_K: a 64-wide K stage is nibble group g = (k0 % 256) / 64 of superblock
// k0 / 256; thread t dequantises sub-block 2g + (t & 1) of row t >> 1.
struct GemmQ4K {
    static constexpr int BLOCK_VALUES = 256;
    static constexpr int BLOCK_BYTES = 144;
    static constexpr int ALIGN = 16;
    static constexpr int STORE_STEP = 0, STORE_STEP_256 = 0;
    struct Raw {
        uint4 hdr, q0, q1;
    };
    template <bool GATED>
    __device__ static __forceinline__ void load(const GemmArgs& a, uint32_t n0, uint32_t k0, Raw& r) {
        const uint32_t t = threadIdx.x;
        const uint8_t* p = gemm_w_row<GATED>(a, n0, t >> 1) + (size_t)(k0 / 256) * 144;
        const uint32_t g = (k0 % 256) / 64;
        r.hdr = load_u4(p);
        r.q0 = load_u4(p + 16 + g * 32);
        r.q1 = load_u4(p + 32 + g * 32);
    }
    __device__ static __forceinline__ void store(const Raw& r, uint16_t* lds_b, uint32_t k0) {
        const uint32_t t = threadIdx.x;
        const uint32_t g = (k0 % 256) / 64;
        const uint32_t j = 2 * g + (t & 1);  // sub-block
        const float d = f16_bits_to_f32(r.hdr.x & 0xffffu);
        const float dmin = f16_bits_to_f32(r.hdr.x >> 16);
        // 6-bit scale/min of sub-block j (12 bytes at 4..15: hdr.y, hdr.z, hdr.w)
        const uint8_t sb[12] = {
            (uint8_t)r.hdr.y, (uint8_t)(r.hdr.y >> 8), (uint8_t)(r.hdr.y >> 16), (uint8_t)(r.hdr.y >> 24),
            (uint8_t)r.hdr.z, (uint8_t)(r.hdr.z >> 8), (uint8_t)(r.hdr.z >> 16), (uint8_t)(r.hdr.z >> 24),
            (uint8_t)r.hdr.w, (uint8_t)(r.hdr.w >> 8), (uint8_t)(r.hdr.w >> 16), (uint8_t)(r.hdr.w >> 24)};
        uint32_t sc, mn;
        if (j < 4) {
            sc = sb[j] & 63u;
            mn = sb[j + 4] & 63u;
        } else {
            sc = (sb[j + 4] & 0xfu) | ((sb[j - 4] >> 6) << 4);
            mn = (sb[j + 4] >> 4) | ((sb[j] >> 6) << 4);
        }
        const float ds = d * (float)sc;
        const float dm = dmin * (float)mn;
        const uint32_t q[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
        const int sh = (t & 1) * 4;  // low nibbles: sub-block 2g, high: 2g+1
        uint32_t o[16];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const uint32_t w = q[c] >> sh;
            const float v0 = ds * (float)(w & 0xfu) - dm;
            const float v1 = ds * (float)((w >> 8) & 0xfu) - dm;
            const float v2 = ds * (float)((w >> 16) & 0xfu) - dm;
            const float v3 = ds * (float)((w >> 24) & 0xfu) - dm;
            o[2 * c] = pack_bf16x2(v0, v1);
            o[2 * c + 1] = pack_bf16x2(v2, v3);
        }
        uint16_t* dst = lds_b + (t >> 1) * GQ_LDS_ROW + (t & 1) * 32;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            *reinterpret_cast<uint4*>(dst + 8 * i) = make_uint4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
    }
};

// Q6_K: a 64-wide K stage is parts p0, p0 + 1 of half h of superblock k0 / 256
// (value 128 h + 32 p + l, l < 32); thread t dequantises part p0 + (t & 1) of
// row t >> 1:  value = (d * sc[8h + 2p + l/16]) * (q - 32),
//   q = (ql[64h + 32(p&1) + l] >> 4(p>>1) & 15) | ((qh[32h + l] >> 2p) & 3) << 4.
// Blocks are 210 B, so only halfword aligned: the 16-B loads are unaligned.
struct GemmQ6K {
    static constexpr int BLOCK_VALUES = 256;
    static constexpr int BLOCK_BYTES = 210;
    static constexpr int ALIGN = 2;
    static constexpr int STORE_STEP = 0, STORE_STEP_256 = 1;  // at 256 rows, 0 spills registers
    struct Raw {
        uint4 ql0, ql1, qh0, qh1;
        uint32_t sc, d;
    };
    template <bool GATED>
    __device__ static __forceinline__ void load(const GemmArgs& a, uint32_t n0, uint32_t k0, Raw& r) {
        const uint32_t t = threadIdx.x;
        const uint8_t* blk = gemm_w_row<GATED>(a, n0, t >> 1) + (size_t)(k0 / 256) * 210;
        const uint32_t h = (k0 % 256) / 128;
        const uint32_t p = (k0 % 128) / 32 + (t & 1);
        const uint8_t* ql = blk + 64 * h + 32 * (p & 1);
        r.ql0 = load_u4_ua(ql);
        r.ql1 = load_u4_ua(ql + 16);
        r.qh0 = load_u4_ua(blk + 128 + 32 * h);
        r.qh1 = load_u4_ua(blk + 128 + 32 * h + 16);
        r.sc = load_u16(blk + 192 + 8 * h + 2 * p);
        r.d = load_u16(blk + 208);
    }
    __device__ static __forceinline__ void store(const Raw& r, uint16_t* lds_b, uint32_t k0) {
        const uint32_t t = threadIdx.x;
        const uint32_t p = (k0 % 128) / 32 + (t & 1);
        const uint32_t shl = 4 * (p >> 1), shh = 2 * p;
        const float d = f16_bits_to_f32(r.d);
        const float a0 = d * (float)(int8_t)(r.sc & 0xffu);  // values l < 16
        const float a1 = d * (float)(int8_t)(r.sc >> 8);     // values l >= 16
        const uint32_t ql[8] = {r.ql0.x, r.ql0.y, r.ql0.z, r.ql0.w, r.ql1.x, r.ql1.y, r.ql1.z, r.ql1.w};
        const uint32_t qh[8] = {r.qh0.x, r.qh0.y, r.qh0.z, r.qh0.w, r.qh1.x, r.qh1.y, r.qh1.z, r.qh1.w};
        uint32_t o[16];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const float a = c < 4 ? a0 : a1;
            float v[4];
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const uint32_t q = ((ql[c] >> (8 * b + shl)) & 15u) | (((qh[c] >> (8 * b + shh)) & 3u) << 4);
                v[b] = a * (float)((int)q - 32);
            }
            o[2 * c] = pack_bf16x2(v[0], v[1]);
            o[2 * c + 1] = pack_bf16x2(v[2], v[3]);
        }
        uint16_t* dst = lds_b + (t >> 1) * GQ_LDS_ROW + (t & 1) * 32;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            *reinterpret_cast<uint4*>(dst + 8 * i) = make_uint4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
    }
};

// bf16 rows (GGUF BF16): no dequantisation, the stage's 64 values of a row copied as they are; thread t
// copies half (t & 1) of row t >> 1.  Weights a prefill pass dequantised once (t2h_dequantize_bf16), or a
// model kept in bf16.
struct GemmBF16 {
    static constexpr int BLOCK_VALUES = 64;
    static constexpr int BLOCK_BYTES = 128;
    static constexpr int ALIGN = 16;
    // measured at M 16384: after step 0 fastest (1: 2-3 % slower, 2: 3 %); tile groups of 8 down M as the
    // other formats (4 and 16: 1-2 % slower)
    static constexpr int STORE_STEP = 0, STORE_STEP_256 = 0;
    struct Raw {
        uint4 v[4];
        bool inside;  // false: a stage past the row's end, stored as zeros
    };
    template <bool GATED>
    __device__ static __forceinline__ void load(const GemmArgs& a, uint32_t n0, uint32_t k0, Raw& r) {
        const uint32_t t = threadIdx.x;
        const uint32_t blk = k0 / 64;
        r.inside = blk < a.w_blocks;
        const uint8_t* p = gemm_w_row<GATED>(a, n0, t >> 1) + (size_t)(r.inside ? blk : a.w_blocks - 1) * 128 +
                           (t & 1) * 64;
#pragma unroll
        for (int i = 0; i < 4; ++i) r.v[i] = load_u4(p + 16 * i);
    }
    __device__ static __forceinline__ void store(const Raw& r, uint16_t* lds_b) {
        const uint32_t t = threadIdx.x;
        uint16_t* dst = lds_b + (t >> 1) * GQ_LDS_ROW + (t & 1) * 32;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            *reinterpret_cast<uint4*>(dst + 8 * i) = r.inside ? r.v[i] : make_uint4(0u, 0u, 0u, 0u);
    }
};

template <class F>
__device__ __forceinline__ void store_w(const typename F::Raw& r, uint16_t* lds_b, uint32_t k0) {
    if constexpr (F::BLOCK_VALUES == 256) {
        F::store(r, lds_b, k0);
    } else {
        F::store(r, lds_b);
    }
}

// ------------------------------------------------------ dequantise once ----

// out[rows, k] bf16 = the values gemm_q_kernel dequantises into its LDS tiles: the same load and store code
// into the same padded LDS rows, then copied out, so a GEMM over `out` (GemmBF16) multiplies bit-identical
// operands.  Block (row tile r0 = 256 blockIdx.x, stage blockIdx.y).
template <class F>
__global__ __launch_bounds__(GQ_THREADS) void gemm_dequant_bf16_kernel(const GemmArgs a, uint16_t* __restrict__ out) {
    __shared__ __align__(16) uint16_t lds_b[GQ_BN * GQ_LDS_ROW];
    const uint32_t n0 = blockIdx.x * GQ_BN, k0 = blockIdx.y * GQ_BK;
    typename F::Raw rw;
    F::template load<false>(a, n0, k0, rw);
    store_w<F>(rw, lds_b, k0);
    __syncthreads();
    const uint32_t t = threadIdx.x;
    const uint32_t row = n0 + (t >> 1);
    if (row >= a.n) return;
    const uint16_t* src = lds_b + (t >> 1) * GQ_LDS_ROW + (t & 1) * 32;
    uint16_t* dst = out + (size_t)row * a.k + k0 + (t & 1) * 32;
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<uint4*>(dst + 8 * i) = *reinterpret_cast<const uint4*>(src + 8 * i);
}

// Q8_0 rows straight to memory: thread i converts block i of the matrix (32 values, 34 B in, 64 B out) with
// GemmQ80::convert, the tile loop's own conversion, with no LDS round trip (each thread writes back only what
// it converted).
__global__ __launch_bounds__(256) void gemm_dequant_q8_0_kernel(const uint8_t* __restrict__ w, uint32_t rows,
                                                                uint32_t blocks_per_row, uint16_t* __restrict__ out) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)rows * blocks_per_row) return;
    const uint8_t* p = w + i * 34;  // rows are whole blocks, so block i of the matrix starts at 34 i
    GemmQ80::Raw r;
    r.d = load_u16(p);
    r.inside = true;
    r.q0 = load_u4_ua(p + 2);
    r.q1 = load_u4_ua(p + 18);
    uint32_t o[16];
    GemmQ80::convert(r, o);
    uint16_t* dst = out + i * 32;  // and the bf16 rows are blocks_per_row * 32 values long
#pragma unroll
    for (int j = 0; j < 4; ++j)
        *reinterpret_cast<uint4*>(dst + 8 * j) = make_uint4(o[4 * j], o[4 * j + 1], o[4 * j + 2], o[4 * j + 3]);
}

template <class F>
static int gemm_dequant_launch(const void* w, uint32_t rows, uint32_t k, void* out, void* stream) {
    if (!w || !out) return T2H_ERR_NULL;
    if (k == 0 || k % GQ_BK != 0 || k % F::BLOCK_VALUES != 0) return T2H_ERR_SHAPE;
    if ((reinterpret_cast<uintptr_t>(w) & (F::ALIGN - 1)) != 0) return T2H_ERR_ALIGN;
    if ((reinterpret_cast<uintptr_t>(out) & 15) != 0) return T2H_ERR_ALIGN;
    if (rows == 0) return T2H_OK;
    GemmArgs a = {};
    a.w = reinterpret_cast<const uint8_t*>(w);
    a.n = rows;
    a.k = k;
    a.w_blocks = k / F::BLOCK_VALUES;
    a.row_bytes = a.w_blocks * F::BLOCK_BYTES;
    if constexpr (std::is_same<F, GemmQ80>::value) {
        const size_t blocks = (size_t)rows * a.w_blocks;
        hipLaunchKernelGGL(gemm_dequant_q8_0_kernel, dim3((unsigned)((blocks + 255) / 256)), dim3(256), 0,
                           reinterpret_cast<hipStream_t>(stream), a.w, rows, a.w_blocks,
                           reinterpret_cast<uint16_t*>(out));
    } else {
        hipLaunchKernelGGL(gemm_dequant_bf16_kernel<F>, dim3((rows + GQ_BN - 1) / GQ_BN, k / GQ_BK),
                           dim3(GQ_THREADS), 0, reinterpret_cast<hipStream_t>(stream), a,
                           reinterpret_cast<uint16_t*>(out));
    }
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}

// ---------------------------------------------------------------- kernel --

// The block's tile: XCD-contiguous runs of blockIdx (blocks are dealt to the 8 XCDs round-robin), then groups
// of GQ_GROUP_M tiles down M.
__device__ __forceinline__ void gemm_tile_of(const GemmArgs& a, uint32_t& tile_m, uint32_t& tile_n) {
    const uint32_t total = a.tiles_m * a.tiles_n;
    uint32_t pid = blockIdx.x;
    if (total % 8 == 0) pid = (pid % 8) * (total / 8) + pid / 8;
    const uint32_t per_group = GQ_GROUP_M * a.tiles_n;
    const uint32_t first_m = (pid / per_group) * GQ_GROUP_M;
    const uint32_t gsize = min(a.tiles_m - first_m, (uint32_t)GQ_GROUP_M);
    tile_m = first_m + (pid % per_group) % gsize;
    tile_n = (pid % per_group) / gsize;
}

// MI = 32-row MFMA tiles per wave down M: 4 gives 256 x 256 block tiles, 2
// gives 128 x 256 for problems with few 256-row tiles.
template <class F, int EPI, int MI>
__global__ __launch_bounds__(GQ_THREADS) void gemm_q_kernel(const GemmArgs a) {
    constexpr int GQ_BM = 64 * MI;
    constexpr int ACH = GQ_BM * GQ_BK / 8 / GQ_THREADS;  // 16-B A chunks per thread
    __shared__ __align__(16) uint16_t lds_a[2][GQ_BM * GQ_LDS_ROW];
    __shared__ __align__(16) uint16_t lds_b[2][GQ_BN * GQ_LDS_ROW];

    uint32_t tile_m, tile_n;
    gemm_tile_of(a, tile_m, tile_n);
    const uint32_t m0 = tile_m * GQ_BM, n0 = tile_n * GQ_BN;

    const uint32_t t = threadIdx.x;
    const int lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int wm = wave >> 2;  // 0..1: rows wm * 32 MI
    const int wn = wave & 3;   // 0..3: cols wn * 64

    // A stage load: GQ_BM rows x 64 bf16 in 16-B chunks, ACH per thread
    // this block's K stages: [kt0, kt0 + KT) (all of K, or split blockIdx.y's part of it)
    uint32_t kt0 = 0, KT = a.k / GQ_BK;
    if (a.split_stages != 0) {
        kt0 = blockIdx.y * a.split_stages;
        KT = min(KT - kt0, a.split_stages);
    }
    uint4 ra[ACH];
    typename F::Raw rw;
    auto load_stage = [&](uint32_t kt) {
        const uint32_t k0 = (kt0 + kt) * GQ_BK;
#pragma unroll
        for (int i = 0; i < ACH; ++i) {
            const uint32_t c = t + GQ_THREADS * i;
            uint32_t row = m0 + (c >> 3);
            row = row < a.m ? row : a.m - 1;
            ra[i] = load_u4(a.a + (size_t)row * a.k + k0 + (c & 7) * 8);
        }
        F::template load<EPI == GQEPI_SWIGLU || EPI == GQEPI_GATED_F32>(a, n0, k0, rw);
    };
    auto store_stage = [&](uint32_t kt, int s) {
#pragma unroll
        for (int i = 0; i < ACH; ++i) {
            const uint32_t c = t + GQ_THREADS * i;
            *reinterpret_cast<uint4*>(&lds_a[s][(c >> 3) * GQ_LDS_ROW + (c & 7) * 8]) = ra[i];
        }
        store_w<F>(rw, lds_b[s], (kt0 + kt) * GQ_BK);
    };
    // part p (0..3) of store_stage: A chunks after MFMA step SS, the weights after the next (the later the
    // step, the longer the global loads issued at the end of the stage before have to land)
    constexpr int SS = MI == 4 ? F::STORE_STEP_256 : F::STORE_STEP;
    auto store_part = [&](int p, uint32_t kt, int s) {
        if (p == SS) {
#pragma unroll
            for (int i = 0; i < ACH; ++i) {
                const uint32_t c = t + GQ_THREADS * i;
                *reinterpret_cast<uint4*>(&lds_a[s][(c >> 3) * GQ_LDS_ROW + (c & 7) * 8]) = ra[i];
            }
        } else if (p == SS + 1) {
            store_w<F>(rw, lds_b[s], (kt0 + kt) * GQ_BK);
        }
    };
    static_assert(SS >= 0 && SS + 1 < GQ_BK / 16, "store steps within the stage");

    f32x16_t acc[MI][2];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    // Stage kt + 1's global loads are issued right after stage kt's LDS store,
    // before the barrier, so they are in flight through the barrier and all of
    // stage kt's matrix work.
    load_stage(0);
    store_stage(0, 0);
    if (KT > 1) load_stage(1);
    __syncthreads();

    const int frag_row = lane & 31;
    const int frag_k = (lane >> 5) * 8;
    // the 16-deep MFMA steps of stage kt from LDS buffer s; part p of the next stage's LDS stores after step p
    auto mma_stage = [&](uint32_t kt, int s, bool store_next) {
        const uint16_t* sa = lds_a[s] + (wm * 32 * MI + frag_row) * GQ_LDS_ROW + frag_k;
        const uint16_t* sb = lds_b[s] + (wn * 64 + frag_row) * GQ_LDS_ROW + frag_k;
#pragma unroll
        for (int kk = 0; kk < GQ_BK; kk += 16) {
            bf16x8_t fa[MI], fb[2];
#pragma unroll
            for (int i = 0; i < MI; ++i)
                fa[i] = *reinterpret_cast<const bf16x8_t*>(sa + i * 32 * GQ_LDS_ROW + kk);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                fb[j] = *reinterpret_cast<const bf16x8_t*>(sb + j * 32 * GQ_LDS_ROW + kk);
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
            if (GQ_SPLIT_STORE && store_next) store_part(kk / 16, kt + 1, s ^ 1);
        }
    };
    // Every stage but the last stores the next one, so the loop body has no branch around the stores and the
    // scheduler can place the dequantisation between the matrix instructions; the load two stages ahead is
    // clamped to the last stage (a re-read that nothing uses) for the same reason.
    for (uint32_t kt = 0; kt + 1 < KT; ++kt) {
        const int s = kt & 1;
        mma_stage(kt, s, true);
        if (!GQ_SPLIT_STORE) store_stage(kt + 1, s ^ 1);
        load_stage(kt + 2 < KT ? kt + 2 : KT - 1);
        __syncthreads();
    }
    mma_stage(KT - 1, (KT - 1) & 1, false);

    // epilogue: lane holds column (lane % 32) of each 32x32 tile, rows 8(e/4) + 4(lane/32) + e%4
    const uint32_t col_base = n0 + wn * 64 + (lane & 31);
    const uint32_t row_base = m0 + wm * 32 * MI + (lane >> 5) * 4;
    if constexpr (EPI == GQEPI_SWIGLU) {
        // tile column j = 0 holds gate, j = 1 up, of feature f
        const uint32_t f = n0 / 2 + wn * 32 + (lane & 31);
        if (f >= a.n_ff) return;
#pragma unroll
        for (int i = 0; i < MI; ++i) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const uint32_t row = row_base + i * 32 + (e >> 2) * 8 + (e & 3);
                if (row < a.m) {
                    // silu(g) = g / (1 + e^-g) on v_exp_f32 and v_rcp_f32 (e^-g overflowing to inf gives 0)
                    const float g = acc[i][0][e];
                    const float sg = g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * g));
                    reinterpret_cast<uint16_t*>(a.c)[(size_t)row * a.n_ff + f] =
                        (uint16_t)f32_to_bf16_bits(sg * acc[i][1][e]);
                }
            }
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint32_t col = col_base + j * 32;
        const float bj = a.bias != nullptr && col < a.n ? a.bias[col] : 0.0f;
#pragma unroll
        for (int i = 0; i < MI; ++i) {
            // the tile's 16 residual values first, then its 16 results, then the 16 stores, each in registers
            // of their own: element by element, the loads (which may alias the output) and the stores
            // serialised on the memory round trip
            float rv[16];
            if constexpr (EPI == GQEPI_RESID) {
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const uint32_t row = row_base + i * 32 + (e >> 2) * 8 + (e & 3);
                    rv[e] = row < a.m && col < a.n ? a.residual[(size_t)row * a.n + col] : 0.0f;
                }
            }
            float ov[16];
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                float v = acc[i][j][e] + bj;
                if (a.act == GQACT_GELU) v = gelu_erf(v);
                ov[e] = EPI == GQEPI_RESID ? rv[e] + v : v;
            }
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const uint32_t row = row_base + i * 32 + (e >> 2) * 8 + (e & 3);
                if (row < a.m && col < a.n) {
                    const size_t idx = (size_t)row * a.n + col;
                    if constexpr (EPI == GQEPI_BF16)
                        reinterpret_cast<uint16_t*>(a.c)[idx] = (uint16_t)f32_to_bf16_bits(ov[e]);
                    else if constexpr (EPI == GQEPI_RESID)
                        reinterpret_cast<float*>(a.c)[idx] = ov[e];
                    else  // fp32 products; split s of a split-K launch writes its own m x n slice
                        reinterpret_cast<float*>(a.c)[(size_t)blockIdx.y * a.m * a.n + idx] = ov[e];
                }
            }
        }
    }
}

// ------------------------------------------- bf16 rows: LDS-DMA ring ----

// The same product over bf16 weight rows (the dequantise-once path) for grids of >= 512 tiles of 256 x 256 (or
// whole rounds of 256) without bias or activation, with nothing to convert between memory and the matrix cores:
//   * 4 waves (2 x 2), each 128 x 128 of the tile: 16 accumulator tiles of 32 x 32 in the AGPRs, so every
//     16-deep step reads 8 operand fragments from LDS for 16 MFMAs (the 8-wave loop reads 6 for 8);
//   * A and W stages go from global memory straight into LDS (global_load_lds_dwordx4, no VGPR round trip,
//     no ds_write), two stages of 64 K, each row 128 B with its 16-B chunks XOR-swizzled by row so that a
//     fragment read of 16 consecutive rows hits 16 distinct 4-bank groups;
//   * one barrier per stage, placed before the stage's last step (whose fragments are already in registers);
//     the next stage's first fragments are read and the stage-after-next's 16 DMA instructions issued, one
//     per MFMA, while that step's 16 MFMAs run;
//   * every step's fragment reads for the next step are interleaved 1 : 1 with its MFMAs.
// The accumulation order per output element is that of gemm_q_kernel (16-deep steps in K order), so both
// produce bit-identical results.  Measured at M 16384, K 4096, N 12288 (fp32 out): 1288-1324 us against
// 1420-1473 us for gemm_q_kernel<GemmBF16> in the same runs.
constexpr int GR_THREADS = 256;
constexpr int GR_ROWB = GQ_BK * 2;            // bytes per LDS row of a stage
constexpr int GR_STAGE = 2 * 256 * GR_ROWB;   // A rows then W rows: 64 KB
constexpr int GR_IPW = 256 * GR_ROWB / 1024 / 4;  // 1-KB DMA instructions per wave per operand and stage

// LDS-DMA of 16 B per lane into lds_addr + 16 * lane.  M0 holds the LDS base; one wait state separates its
// write from the load that reads it.
__device__ __forceinline__ void gr_dma16(const void* g, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds_addr)
                 : "memory", "m0");
}
__device__ __forceinline__ void gr_wait_vm0() { __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8)); }
__device__ __forceinline__ void gr_wait_lgkm0() { __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (3 << 14)); }
// slot of 16-B chunk c in LDS row r is c ^ gr_swizzle(r)
__device__ __forceinline__ uint32_t gr_swizzle(uint32_t r) { return (r & 7) ^ ((r >> 3) & 1); }

template <int EPI>
__global__ __launch_bounds__(GR_THREADS) void gemm_bf16_ring_kernel(const GemmArgs a) {
    constexpr bool GATED = EPI == GQEPI_SWIGLU;
    __shared__ __align__(1024) uint8_t lds[2 * GR_STAGE];

    uint32_t tile_m, tile_n;
    gemm_tile_of(a, tile_m, tile_n);
    const uint32_t m0 = tile_m * 256, n0 = tile_n * GQ_BN;
    const uint32_t t = threadIdx.x;
    const int lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const uint32_t KT = a.k / GQ_BK;
    const uint32_t lds0 = __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)&lds[0]);

    // DMA instruction i of this wave moves rows 8 (wave IPW + i) .. + 7 of a stage: lane l brings chunk
    // (l % 8) ^ swizzle(row) of row (l / 8), so LDS slot l % 8 of the row holds it
    const uint8_t* src_a[GR_IPW];
    const uint8_t* src_w[GR_IPW];
#pragma unroll
    for (int i = 0; i < GR_IPW; ++i) {
        const uint32_t r = 8 * (wave * GR_IPW + i) + (lane >> 3);
        const uint32_t c = (lane & 7) ^ gr_swizzle(r);
        const uint32_t row = min(m0 + r, a.m - 1);
        src_a[i] = reinterpret_cast<const uint8_t*>(a.a + (size_t)row * a.k) + c * 16;
        src_w[i] = gemm_w_row<GATED>(a, n0, r) + c * 16;
    }
    const uint32_t dma_base = lds0 + wave * GR_IPW * 1024;

    f32x16_t acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    const uint32_t fr = lane & 31, fh = lane >> 5;
    const uint32_t swz = gr_swizzle(fr);  // rows of a fragment start at multiples of 32
    const uint32_t off_a = (wm * 128 + fr) * GR_ROWB, off_w = 256 * GR_ROWB + (wn * 128 + fr) * GR_ROWB;
    bf16x8_t fa[2][4], fb[2][4];
    auto read_step = [&](uint32_t buf, int step, int b) {
        const uint8_t* st = lds + buf * GR_STAGE;
        const uint32_t slot = ((step * 2 + fh) ^ swz) * 16;
#pragma unroll
        for (int i = 0; i < 4; ++i) fa[b][i] = *reinterpret_cast<const bf16x8_t*>(st + off_a + i * 32 * GR_ROWB + slot);
#pragma unroll
        for (int j = 0; j < 4; ++j) fb[b][j] = *reinterpret_cast<const bf16x8_t*>(st + off_w + j * 32 * GR_ROWB + slot);
    };
    auto issue_stage = [&](uint32_t kt, uint32_t buf) {
        const uint32_t kb = kt * GR_ROWB;
#pragma unroll
        for (int i = 0; i < GR_IPW; ++i) gr_dma16(src_a[i] + kb, dma_base + buf * GR_STAGE + i * 1024);
#pragma unroll
        for (int i = 0; i < GR_IPW; ++i)
            gr_dma16(src_w[i] + kb, dma_base + buf * GR_STAGE + 256 * GR_ROWB + i * 1024);
    };
    // one 16-deep step: the next step's 8 fragment reads interleaved with the 16 MFMAs
    auto mma_step = [&](int b) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[b][i], fb[b][j], acc[i][j], 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
    };
    // a stage's last step, with DMA instruction q of stage kt's load into buffer buf after MFMA q
    auto mma_step_dma = [&](int b, uint32_t kt, uint32_t buf) {
        const uint32_t kb = kt * GR_ROWB;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[b][i], fb[b][j], acc[i][j], 0, 0, 0);
                const int q = i * 4 + j;
                if (q < GR_IPW)
                    gr_dma16(src_a[q] + kb, dma_base + buf * GR_STAGE + q * 1024);
                else
                    gr_dma16(src_w[q - GR_IPW] + kb, dma_base + buf * GR_STAGE + 256 * GR_ROWB + (q - GR_IPW) * 1024);
            }
    };
    static_assert(2 * GR_IPW == 16, "one DMA instruction per MFMA of a step");

    // Stage kt lives in buffer kt % 2.  Every iteration issues one stage's DMA, clamped to the last stage past
    // the end (into a buffer nothing reads again), so the wait before each barrier is the same.
    issue_stage(0, 0);
    gr_wait_vm0();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    issue_stage(min(1u, KT - 1), 1);
    read_step(0, 0, 0);
    constexpr int STEPS = GQ_BK / 16;
    for (uint32_t kt = 0; kt + 1 < KT; ++kt) {
        const uint32_t buf = kt & 1;
#pragma unroll
        for (int step = 0; step + 1 < STEPS; ++step) {
            read_step(buf, step + 1, (step + 1) & 1);
            mma_step(step & 1);
        }
        // stage kt + 1 landed (every wave's DMA), stage kt's reads done (every wave): buffer buf is free
        gr_wait_vm0();
        gr_wait_lgkm0();
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        read_step(buf ^ 1, 0, 0);
        mma_step_dma((STEPS - 1) & 1, min(kt + 2, KT - 1), buf);
    }
    {
        const uint32_t buf = (KT - 1) & 1;
#pragma unroll
        for (int step = 0; step + 1 < STEPS; ++step) {
            read_step(buf, step + 1, (step + 1) & 1);
            mma_step(step & 1);
        }
        mma_step((STEPS - 1) & 1);
    }
    gr_wait_vm0();  // the clamped DMA of the last iteration lands before the block's LDS is released

    // epilogue: lane holds column (lane % 32) of each 32 x 32 tile, rows 8 (e / 4) + 4 (lane / 32) + e % 4
    const uint32_t row_base = m0 + wm * 128 + (lane >> 5) * 4;
    if constexpr (EPI == GQEPI_SWIGLU) {
        // tile columns j = 2 p hold gate and j = 2 p + 1 up of feature f = f0 + 32 p; the two features of a row
        // are stored back to back, so each 128-B line of the output is written whole
        const uint32_t f0 = n0 / 2 + wn * 64 + (lane & 31);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const uint32_t row = row_base + i * 32 + (e >> 2) * 8 + (e & 3);
#pragma unroll
                for (int p = 0; p < 2; ++p) {
                    const uint32_t f = f0 + p * 32;
                    if (row < a.m && f < a.n_ff) {
                        const float g = acc[i][2 * p][e];
                        const float sg =
                            g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * g));
                        reinterpret_cast<uint16_t*>(a.c)[(size_t)row * a.n_ff + f] =
                            (uint16_t)f32_to_bf16_bits(sg * acc[i][2 * p + 1][e]);
                    }
                }
            }
        return;
    }
    const uint32_t col0 = n0 + wn * 128 + (lane & 31);
    if constexpr (EPI == GQEPI_BF16) {
        // a row's 4 tile columns (2 x 128 B) stored back to back
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const uint32_t row = row_base + i * 32 + (e >> 2) * 8 + (e & 3);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t col = col0 + j * 32;
                    if (row < a.m && col < a.n)
                        reinterpret_cast<uint16_t*>(a.c)[(size_t)row * a.n + col] =
                            (uint16_t)f32_to_bf16_bits(acc[i][j][e]);
                }
            }
        return;
    }
    if constexpr (EPI == GQEPI_RESID) {
        // fp32 plus the residual, which may be the output itself: the compiler keeps every load behind the
        // stores before it in program order, so the residuals of column group j + 1 (4 x 16 values a lane) are
        // loaded before group j's results are stored, one group ahead (each element is still read before it
        // is written, by the same lane).  Loaded just before each 16 stores, the loads of a tile made 16 round
        // trips one after another.
        // Buffer loads: a lane offset and a scalar offset per element, so the 64 loads in flight need no
        // address registers; rows past M read as zeros (the resource's range), columns past N are not stored.
        float rv[2][4][16];
        const uint64_t mn4 = (uint64_t)a.m * a.n * 4u;
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(a.residual), (short)0, (int)(mn4 < 0x7fffffffu ? mn4 : 0x7fffffffu), 0x00020000);
        const uint32_t lane_off = (row_base * a.n + col0) * 4u;
        auto load_group = [&](int j, float (&r)[4][16]) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const uint32_t el = (uint32_t)(i * 32 + (e >> 2) * 8 + (e & 3)) * a.n + (uint32_t)j * 32;
                    r[i][e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, lane_off, el * 4u, 0));
                }
        };
        load_group(0, rv[0]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (j + 1 < 4) load_group(j + 1, rv[(j + 1) & 1]);
            const uint32_t col = col0 + j * 32;
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const uint32_t row = row_base + i * 32 + (e >> 2) * 8 + (e & 3);
                    if (row < a.m && col < a.n)
                        reinterpret_cast<float*>(a.c)[(size_t)row * a.n + col] = rv[j & 1][i][e] + acc[i][j][e];
                }
        }
        return;
    }
    // fp32 (a tile column is a whole 128-B line per row)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t col = col0 + j * 32;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float rv[16];
            if constexpr (EPI == GQEPI_RESID) {
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const uint32_t row = row_base + i * 32 + (e >> 2) * 8 + (e & 3);
                    rv[e] = row < a.m && col < a.n ? a.residual[(size_t)row * a.n + col] : 0.0f;
                }
            }
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const uint32_t row = row_base + i * 32 + (e >> 2) * 8 + (e & 3);
                if (row < a.m && col < a.n)
                    reinterpret_cast<float*>(a.c)[(size_t)row * a.n + col] =
                        EPI == GQEPI_RESID ? rv[e] + acc[i][j][e] : acc[i][j][e];
            }
        }
    }
}

template <class F, int EPI>
static void gemm_q_dispatch(GemmArgs a, hipStream_t s) {
    const dim3 block(GQ_THREADS);
    a.tiles_n = (a.n + GQ_BN - 1) / GQ_BN;
    // 256-row tiles for big grids; below ~4 tiles per CU the 128-row tile's
    // finer load balance wins over the bigger tile's operand reuse (measured)
    const uint32_t tiles_256 = (a.m + 255) / 256 * a.tiles_n;
    if constexpr (std::is_same<F, GemmBF16>::value && EPI != GQEPI_GATED_F32) {
        // bf16 rows over all of K in one pass: the LDS-DMA ring kernel (256 x 256 tiles, one block per CU) from
        // two rounds of tiles, or from one when the tiles fill whole rounds; a partial round of these large tiles
        // loses to the 128-row loop (measured at M 6000-16384: 288 tiles 3 % slower, 384 equal, 512 11 % and 576
        // 12 % faster, 256 17 % faster)
        const bool whole_rounds = tiles_256 >= 256 && tiles_256 % 256 == 0;
        // (the residual epilogue addresses the residual with 32-bit byte offsets)
        const bool resid_fits = EPI != GQEPI_RESID || (uint64_t)a.m * a.n * 4u < 0x80000000ull;
        if ((tiles_256 >= 512 || whole_rounds) && a.split_stages == 0 && a.w_blocks * GQ_BK == a.k &&
            a.bias == nullptr && a.act == GQACT_NONE && resid_fits) {
            a.tiles_m = (a.m + 255) / 256;
            hipLaunchKernelGGL((gemm_bf16_ring_kernel<EPI>), dim3(a.tiles_m * a.tiles_n), dim3(GR_THREADS), 0, s, a);
            return;
        }
    }
    if (tiles_256 < 1024 && a.m > 128) {
        a.tiles_m = (a.m + 127) / 128;
        hipLaunchKernelGGL((gemm_q_kernel<F, EPI, 2>), dim3(a.tiles_m * a.tiles_n), block, 0, s, a);
    } else {
        a.tiles_m = (a.m + 255) / 256;
        hipLaunchKernelGGL((gemm_q_kernel<F, EPI, 4>), dim3(a.tiles_m * a.tiles_n), block, 0, s, a);
    }
}

// k: the A row length (% 64); w_k: the weight rows' quantized length (<= k,
// whole blocks); columns of A past w_k multiply zeros.
template <class F>
static int gemm_q_launch(const void* x, const void* w, const float* bias, int act, void* y, int out_dtype,
                         const float* residual, uint32_t m, uint32_t k, uint32_t n, uint32_t w_k, void* stream) {
    if (!x || !w || !y) return T2H_ERR_NULL;
    if (k == 0 || k % GQ_BK != 0) return T2H_ERR_SHAPE;
    if (w_k == 0 || w_k > k || w_k % F::BLOCK_VALUES != 0) return T2H_ERR_SHAPE;
    if (F::BLOCK_VALUES == 256 && w_k != k) return T2H_ERR_SHAPE;
    if (act != GQACT_NONE && act != GQACT_GELU) return T2H_ERR_ARG;
    if ((reinterpret_cast<uintptr_t>(x) & 15) != 0) return T2H_ERR_ALIGN;
    if ((reinterpret_cast<uintptr_t>(w) & (F::ALIGN - 1)) != 0) return T2H_ERR_ALIGN;
    int epi;
    if (residual) {
        if (out_dtype != T2H_DTYPE_F32) return T2H_ERR_DTYPE;
        epi = GQEPI_RESID;
    } else if (out_dtype == T2H_DTYPE_F32) {
        epi = GQEPI_F32;
    } else if (out_dtype == T2H_DTYPE_BF16) {
        epi = GQEPI_BF16;
    } else {
        return T2H_ERR_DTYPE;
    }
    if (m == 0 || n == 0) return T2H_OK;
    if ((uint64_t)(m / 128 + 1) * (n / GQ_BN + 1) > 0x7fffffffu) return T2H_ERR_SHAPE;
    GemmArgs a = {};
    a.a = reinterpret_cast<const uint16_t*>(x);
    a.w = reinterpret_cast<const uint8_t*>(w);
    a.c = y;
    a.residual = residual;
    a.bias = bias;
    a.act = act;
    a.m = m;
    a.n = n;
    a.k = k;
    a.w_blocks = w_k / F::BLOCK_VALUES;
    a.row_bytes = a.w_blocks * F::BLOCK_BYTES;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    switch (epi) {
        case GQEPI_F32: gemm_q_dispatch<F, GQEPI_F32>(a, s); break;
        case GQEPI_BF16: gemm_q_dispatch<F, GQEPI_BF16>(a, s); break;
        default: gemm_q_dispatch<F, GQEPI_RESID>(a, s); break;
    }
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}

// ---------------------------------------------------------------- split-K ----

// out = epilogue(sum over the splits of partial[s]) in split order.  Plain: y[row][col] from partial column
// col, + bias, GELU, then fp32 (+ residual) or bf16.  SwiGLU (n_ff > 0): feature f's gate and up products are
// the tile-interleaved columns the gated kernel writes (per 256-column tile: 4 groups of 32 gate then 32 up
// columns, 128 features; partial rows are whole tiles, n_cols a multiple of 256).
__global__ __launch_bounds__(256) void gemm_splitk_reduce_kernel(const float* __restrict__ partial, uint32_t splits,
                                                                 uint32_t m, uint32_t n_cols, uint32_t n_out,
                                                                 uint32_t n_ff, const float* bias, int act,
                                                                 void* y, int out_dtype, const float* residual) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)m * n_out) return;
    const uint32_t row = (uint32_t)(i / n_out), col = (uint32_t)(i % n_out);
    const size_t slice = (size_t)m * n_cols;
    if (n_ff != 0) {
        const uint32_t gc = (col / 128) * 256 + ((col % 128) / 32) * 64 + col % 32;
        const float* pg = partial + (size_t)row * n_cols + gc;
        float g = 0.0f, u = 0.0f;
        for (uint32_t s = 0; s < splits; ++s) {
            g += pg[s * slice];
            u += pg[s * slice + 32];
        }
        const float sg = g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * g));
        reinterpret_cast<uint16_t*>(y)[i] = (uint16_t)f32_to_bf16_bits(sg * u);
        return;
    }
    const float* p = partial + (size_t)row * n_cols + col;
    float v = 0.0f;
    for (uint32_t s = 0; s < splits; ++s) v += p[s * slice];
    v += bias != nullptr ? bias[col] : 0.0f;
    if (act == GQACT_GELU) v = gelu_erf(v);
    if (residual != nullptr)
        reinterpret_cast<float*>(y)[i] = residual[i] + v;
    else if (out_dtype == T2H_DTYPE_F32)
        reinterpret_cast<float*>(y)[i] = v;
    else
        reinterpret_cast<uint16_t*>(y)[i] = (uint16_t)f32_to_bf16_bits(v);
}

// Partial products of `splits` parts of K, then the reduction.  Gated: w_up != nullptr, n = n_ff features.
template <class F>
static int gemm_splitk_launch(const void* x, const void* w, const void* w_up, const float* bias, int act, void* y,
                              int out_dtype, const float* residual, uint32_t m, uint32_t k, uint32_t n, uint32_t w_k,
                              uint32_t splits, void* partials, size_t partials_bytes, void* stream) {
    if (!x || !w || !y || !partials) return T2H_ERR_NULL;
    const bool gated = w_up != nullptr;
    if (k == 0 || k % GQ_BK != 0) return T2H_ERR_SHAPE;
    if (w_k == 0 || w_k > k || w_k % F::BLOCK_VALUES != 0) return T2H_ERR_SHAPE;
    if ((F::BLOCK_VALUES == 256 || gated) && w_k != k) return T2H_ERR_SHAPE;
    if (act != GQACT_NONE && act != GQACT_GELU) return T2H_ERR_ARG;
    if (gated && (bias || act != GQACT_NONE || residual || out_dtype != T2H_DTYPE_BF16)) return T2H_ERR_ARG;
    if (residual && out_dtype != T2H_DTYPE_F32) return T2H_ERR_DTYPE;
    if (out_dtype != T2H_DTYPE_F32 && out_dtype != T2H_DTYPE_BF16) return T2H_ERR_DTYPE;
    if ((reinterpret_cast<uintptr_t>(x) & 15) != 0) return T2H_ERR_ALIGN;
    if (((reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(w_up)) & (F::ALIGN - 1)) != 0)
        return T2H_ERR_ALIGN;
    if ((reinterpret_cast<uintptr_t>(partials) & 15) != 0) return T2H_ERR_ALIGN;
    const uint32_t stages = k / GQ_BK;
    if (splits == 0 || splits > stages || splits > 64) return T2H_ERR_ARG;
    if (m == 0 || n == 0) return T2H_OK;
    if (n > 0x3fffffffu || (uint64_t)m * n > 0x7fffffffu) return T2H_ERR_SHAPE;
    // gated: whole 256-column tiles of gate | up groups, so that every feature's up column exists
    const uint32_t n_cols = gated ? (2 * n + GQ_BN - 1) / GQ_BN * GQ_BN : n;
    if (partials_bytes < t2h_gemm_splitk_bytes(m, n, splits, gated ? 1 : 0)) return T2H_ERR_WORKSPACE;
    GemmArgs a = {};
    a.a = reinterpret_cast<const uint16_t*>(x);
    a.w = reinterpret_cast<const uint8_t*>(w);
    a.w_up = reinterpret_cast<const uint8_t*>(w_up);
    a.c = partials;
    a.m = m;
    a.n = n_cols;
    a.n_ff = gated ? n : 0;
    a.k = k;
    a.w_blocks = w_k / F::BLOCK_VALUES;
    a.row_bytes = a.w_blocks * F::BLOCK_BYTES;
    // every split takes the same number of stages, so none is empty
    const uint32_t per = (stages + splits - 1) / splits;
    a.split_stages = per;
    const uint32_t used = (stages + per - 1) / per;
    a.tiles_n = (n_cols + GQ_BN - 1) / GQ_BN;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    // 128-row tiles as in gemm_q_dispatch, and for up to 128 rows (a 256-row tile would compute half of it for
    // nothing)
    if ((m + 255) / 256 * a.tiles_n < 1024) {
        a.tiles_m = (m + 127) / 128;
        if (gated)
            hipLaunchKernelGGL((gemm_q_kernel<F, GQEPI_GATED_F32, 2>), dim3(a.tiles_m * a.tiles_n, used), dim3(512),
                               0, s, a);
        else
            hipLaunchKernelGGL((gemm_q_kernel<F, GQEPI_F32, 2>), dim3(a.tiles_m * a.tiles_n, used), dim3(512), 0, s,
                               a);
    } else {
        a.tiles_m = (m + 255) / 256;
        if (gated)
            hipLaunchKernelGGL((gemm_q_kernel<F, GQEPI_GATED_F32, 4>), dim3(a.tiles_m * a.tiles_n, used), dim3(512),
                               0, s, a);
        else
            hipLaunchKernelGGL((gemm_q_kernel<F, GQEPI_F32, 4>), dim3(a.tiles_m * a.tiles_n, used), dim3(512), 0, s,
                               a);
    }
    T2H_LAUNCH_CHECK();
    const size_t outs = (size_t)m * n;
    hipLaunchKernelGGL(gemm_splitk_reduce_kernel, dim3((unsigned)((outs + 255) / 256)), dim3(256), 0, s,
                       reinterpret_cast<const float*>(partials), used, m, n_cols, n, a.n_ff, bias, act, y, out_dtype,
                       residual);
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}

}  // namespace t2h

using namespace t2h;

extern "C" int t2h_q8_0_gemm(const void* x, const void* w, void* y, int out_dtype, const float* residual, uint32_t m,
                             uint32_t k, uint32_t n, void* stream) {
    return gemm_q_launch<GemmQ80>(x, w, nullptr, GQACT_NONE, y, out_dtype, residual, m, k, n, k, stream);
}

extern "C" int t2h_q4k_gemm(const void* x, const void* w, void* y, int out_dtype, const float* residual, uint32_t m,
                            uint32_t k, uint32_t n, void* stream) {
    return gemm_q_launch<GemmQ4K>(x, w, nullptr, GQACT_NONE, y, out_dtype, residual, m, k, n, k, stream);
}

extern "C" int t2h_q8_0_linear(const void* x, const void* w, const float* bias, int act, void* y, int out_dtype,
                               const float* residual, uint32_t m, uint32_t k, uint32_t n, uint32_t w_k,
                               void* stream) {
    return gemm_q_launch<GemmQ80>(x, w, bias, act, y, out_dtype, residual, m, k, n, w_k, stream);
}

extern "C" int t2h_bf16_gemm(const void* x, const void* w, void* y, int out_dtype, const float* residual,
                             uint32_t m, uint32_t k, uint32_t n, void* stream) {
    return gemm_q_launch<GemmBF16>(x, w, nullptr, GQACT_NONE, y, out_dtype, residual, m, k, n, k, stream);
}

extern "C" int t2h_bf16_linear(const void* x, const void* w, const float* bias, int act, void* y, int out_dtype,
                               const float* residual, uint32_t m, uint32_t k, uint32_t n, void* stream) {
    return gemm_q_launch<GemmBF16>(x, w, bias, act, y, out_dtype, residual, m, k, n, k, stream);
}

extern "C" int t2h_dequantize_bf16(int wtype, const void* w, uint32_t rows, uint32_t k, void* out, void* stream) {
    switch (wtype) {
        case T2H_WTYPE_Q8_0: return gemm_dequant_launch<GemmQ80>(w, rows, k, out, stream);
        case T2H_WTYPE_Q4_K: return gemm_dequant_launch<GemmQ4K>(w, rows, k, out, stream);
        case T2H_WTYPE_Q6_K: return gemm_dequant_launch<GemmQ6K>(w, rows, k, out, stream);
        default: return T2H_ERR_DTYPE;
    }
}

extern "C" int t2h_q6k_gemm(const void* x, const void* w, void* y, int out_dtype, const float* residual, uint32_t m,
                            uint32_t k, uint32_t n, void* stream) {
    return gemm_q_launch<GemmQ6K>(x, w, nullptr, GQACT_NONE, y, out_dtype, residual, m, k, n, k, stream);
}

// y[m, n_ff] = bf16(silu(x . deq(W_gate)^T) * (x . deq(W_up)^T)): the prefill MLP's gate and up products
// in one launch, SwiGLU applied in the epilogue (no fp32 gate/up intermediates).
template <class F>
static int gemm_swiglu_launch(const void* x, const void* w_gate, const void* w_up, void* y, uint32_t m, uint32_t k,
                              uint32_t n_ff, void* stream) {
    if (!x || !w_gate || !w_up || !y) return T2H_ERR_NULL;
    if (k == 0 || k % GQ_BK != 0 || k % F::BLOCK_VALUES != 0) return T2H_ERR_SHAPE;
    if ((reinterpret_cast<uintptr_t>(x) & 15) != 0) return T2H_ERR_ALIGN;
    if (((reinterpret_cast<uintptr_t>(w_gate) | reinterpret_cast<uintptr_t>(w_up)) & (F::ALIGN - 1)) != 0)
        return T2H_ERR_ALIGN;
    if (n_ff > 0x3fffffffu) return T2H_ERR_SHAPE;
    if (m == 0 || n_ff == 0) return T2H_OK;
    GemmArgs a = {};
    a.a = reinterpret_cast<const uint16_t*>(x);
    a.w = reinterpret_cast<const uint8_t*>(w_gate);
    a.w_up = reinterpret_cast<const uint8_t*>(w_up);
    a.c = y;
    a.m = m;
    a.k = k;
    a.n_ff = n_ff;
    a.n = 2 * n_ff;
    a.w_blocks = k / F::BLOCK_VALUES;
    a.row_bytes = a.w_blocks * F::BLOCK_BYTES;
    gemm_q_dispatch<F, GQEPI_SWIGLU>(a, reinterpret_cast<hipStream_t>(stream));
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}

extern "C" size_t t2h_gemm_splitk_bytes(uint32_t m, uint32_t n, uint32_t splits, int swiglu) {
    const size_t n_cols = swiglu ? ((size_t)2 * n + GQ_BN - 1) / GQ_BN * GQ_BN : n;
    return (size_t)splits * m * n_cols * sizeof(float);
}

extern "C" int t2h_gemm_splitk(int wtype, const void* x, const void* w, const void* w_up, const float* bias, int act,
                               void* y, int out_dtype, const float* residual, uint32_t m, uint32_t k, uint32_t n,
                               uint32_t w_k, uint32_t splits, void* partials, size_t partials_bytes, void* stream) {
    switch (wtype) {
        case T2H_WTYPE_Q8_0:
            return gemm_splitk_launch<GemmQ80>(x, w, w_up, bias, act, y, out_dtype, residual, m, k, n, w_k, splits,
                                               partials, partials_bytes, stream);
        case T2H_WTYPE_Q4_K:
            return gemm_splitk_launch<GemmQ4K>(x, w, w_up, bias, act, y, out_dtype, residual, m, k, n, w_k, splits,
                                               partials, partials_bytes, stream);
        case T2H_WTYPE_Q6_K:
            return gemm_splitk_launch<GemmQ6K>(x, w, w_up, bias, act, y, out_dtype, residual, m, k, n, w_k, splits,
                                               partials, partials_bytes, stream);
        case T2H_WTYPE_BF16:
            return gemm_splitk_launch<GemmBF16>(x, w, w_up, bias, act, y, out_dtype, residual, m, k, n, w_k, splits,
                                                partials, partials_bytes, stream);
        default: return T2H_ERR_DTYPE;
    }
}

extern "C" int t2h_gemm_swiglu(int wtype, const void* x, const void* w_gate, const void* w_up, void* y, uint32_t m,
                               uint32_t k, uint32_t n_ff, void* stream) {
    switch (wtype) {
        case T2H_WTYPE_Q8_0: return gemm_swiglu_launch<GemmQ80>(x, w_gate, w_up, y, m, k, n_ff, stream);
        case T2H_WTYPE_Q4_K: return gemm_swiglu_launch<GemmQ4K>(x, w_gate, w_up, y, m, k, n_ff, stream);
        case T2H_WTYPE_Q6_K: return gemm_swiglu_launch<GemmQ6K>(x, w_gate, w_up, y, m, k, n_ff, stream);
        case T2H_WTYPE_BF16: return gemm_swiglu_launch<GemmBF16>(x, w_gate, w_up, y, m, k, n_ff, stream);
        default: return T2H_ERR_DTYPE;
    }
}
