// tile_store.h -- shared pieces of the 256x256-tile persistent GEMMs
// (gemm_big.hip, gemm_packed.hip): the XCD-aware tile order, the per-tile
// bias prefetch and the epilogue that writes a finished tile straight from
// the MFMA accumulators.
//
// Tile layout: 4 waves, wave (wm, wn) owns rows wm*128.. and logical columns
// wn*128.. of the tile as 4x4 fragments of 32x32 (v_mfma_f32_32x32x16_f16).
// D[i][j] of a fragment sits in lane j + 32*((i/4)%2), register
// (i%4) + 4*(i/8). Gated tiles cover 128 outputs: wave column wn owns outputs
// wn*64.., its fragments 0-1 hold the gate rows and 2-3 the matching up rows.
#pragma once
#include <algorithm>
#include <type_traits>

#include "device_common.h"
#include "kernels.h"

namespace vai_dev {

// Launch-order index L -> (tm, tn). Workgroup b runs on XCD b % 8 and walks
// L = b, b + G, ... (G % 8 == 0), so the tiles resident on one XCD at a time
// (8 M-tiles x 4 N-tiles at the config-3 shape) share A and B in its L2.
struct TileOrder {
    uint32_t tiles_m, tiles_n;
    bool xcd;
    __host__ __device__ __forceinline__ void of(uint32_t L, uint32_t& tm, uint32_t& tn) const
    {
        if (xcd) {
            const uint32_t x = L % 8, local = L / 8;
            tm = local % tiles_m;
            tn = x * (tiles_n / 8) + local / tiles_m;
        } else {
            tm = L % tiles_m;
            tn = L / tiles_m;
        }
    }
    __host__ __device__ static TileOrder make(uint32_t tiles_m, uint32_t tiles_n, uint32_t grid)
    {
        TileOrder o;
        o.tiles_m = tiles_m;
        o.tiles_n = tiles_n;
        o.xcd = grid % 8 == 0 && (tiles_m * tiles_n) % 8 == 0 && tiles_m <= 8 && 8 % tiles_m == 0 && tiles_n % 8 == 0;
        return o;
    }
};

// The accumulators are read through this so that the register allocator
// keeps them in AGPRs across the tile loop (a plain VALU use of an MFMA
// result lets it move accumulators into VGPRs and spill). The asm is opaque
// to the compiler's hazard checks: tile_store pads the MFMA -> read distance.
__device__ __forceinline__ float agpr_read(float a)
{
    float v;
    asm("v_accvgpr_read_b32 %0, %1" : "=v"(v) : "a"(a));
    return v;
}

// A row bias for the tile's columns, loaded before the tile's K loop so that
// the loads are long complete when the epilogue reads them (a load still in
// flight at the epilogue makes the compiler wait for every copy issued after
// it). Gated: [0..1] the gate bias of fragment columns 0-1, [2..3] the up bias.
template <bool GATED>
__device__ __forceinline__ void tile_col_bias(const GemmParams& p, uint32_t tn, int wn, int fr, float (&cb)[4])
{
#pragma unroll
    for (int j = 0; j < 4; ++j) cb[j] = 0.f;
    if constexpr (GATED) {
        const uint32_t H = p.H, col0 = tn * 128 + wn * 64 + fr;
        if (p.bias) {
#pragma unroll
            for (int jj = 0; jj < 2; ++jj)
                if (col0 + jj * 32 < H) {
                    cb[jj] = ld(p.bias, p.bias_dtype, col0 + jj * 32);
                    cb[jj + 2] = ld(p.bias, p.bias_dtype, H + col0 + jj * 32);
                }
        }
    } else {
        const uint32_t N = p.N, col0 = tn * 256 + wn * 128 + fr;
        if (p.bias && p.bias_repeat == N) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (col0 + j * 32 < N) cb[j] = ld(p.bias, p.bias_dtype, col0 + j * 32);
        }
    }
}

// Activation with a compile-time kind; kind 6 = the runtime kind `epi`.
template <uint32_t EPI>
__device__ __forceinline__ float act(float x, uint32_t epi)
{
    return epilogue(x, EPI == 6 ? epi : EPI);
}

// Writes tile (tm, tn) from the accumulators. For each register a half-wave
// holds 32 consecutive columns of one row, so each store instruction writes
// two 128-byte row segments.
//
// Fast path (fp32 output, the tile's columns inside the output, a bias that
// is one row): buffer stores from a resource that starts at the tile's first
// row and ends at the output's last row, so rows past M are dropped by the
// hardware bounds check and no output needs a test; the common activations
// are compile-time. Other tiles and outputs go through a per-output path.
template <bool GATED, uint32_t EPI>
__device__ __forceinline__ void tile_store_fast(const GemmParams& p, float16v (&acc)[4][4], const float (&cb)[4],
                                                uint32_t tm, uint32_t tn, int wm, int wn, int fr, int fk)
{
    const uint32_t ld_out = GATED ? p.H : p.N;   // output row length
    const uint32_t rows_left = p.M - tm * 256;
    const __amdgpu_buffer_rsrc_t out = __builtin_amdgcn_make_buffer_rsrc(
        (void*)((float*)p.C + (size_t)tm * 256 * ld_out), (short)0,
        (int)std::min<size_t>((size_t)rows_left * ld_out * 4, 0x7FFFFFFF), 0x00020000);
    const uint32_t col0 = GATED ? tn * 128 + wn * 64 + fr : tn * 256 + wn * 128 + fr;
    const uint32_t lane_off = ((wm * 128 + 4 * fk) * ld_out + col0) * 4;
    const uint32_t row_bytes = ld_out * 4;
    const uint32_t epi = p.epilogue;
    const float s = p.scalar_scale;
    constexpr int JN = GATED ? 2 : 4;
    static_for<4>([&](auto I) __attribute__((always_inline)) {
        static_for<JN>([&](auto J) __attribute__((always_inline)) {
            constexpr int i = I, j = J;
            static_for<16>([&](auto R) __attribute__((always_inline)) {
                constexpr int rr = R;
                float v;
                if constexpr (GATED)
                    v = act<EPI>(agpr_read(acc[i][j][rr]) + cb[j], epi) * (agpr_read(acc[i][j + 2][rr]) + cb[j + 2]);
                else
                    v = s * act<EPI>(agpr_read(acc[i][j][rr]) + cb[j], epi);
                const uint32_t voff = lane_off + (uint32_t)(i * 32 + (rr % 4) + 8 * (rr / 4)) * row_bytes + j * 128;
                __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), out, (int)voff, 0, 0);
            });
            __builtin_amdgcn_sched_barrier(0);   // 16 outputs at a time: few live registers
        });
    });
}

template <bool GATED>
__device__ __forceinline__ void tile_store_any(const GemmParams& p, float16v (&acc)[4][4], const float (&cb)[4],
                                               uint32_t tm, uint32_t tn, int wm, int wn, int fr, int fk)
{
    const uint32_t M = p.M, row0 = tm * 256 + wm * 128 + 4 * fk;
    if constexpr (GATED) {
        const uint32_t H = p.H, col0 = tn * 128 + wn * 64 + fr;
        static_for<4>([&](auto I) __attribute__((always_inline)) {
            static_for<2>([&](auto JJ) __attribute__((always_inline)) {
                static_for<16>([&](auto R) __attribute__((always_inline)) {
                    constexpr int i = I, jj = JJ, rr = R;
                    const uint32_t row = row0 + i * 32 + (rr % 4) + 8 * (rr / 4), col = col0 + jj * 32;
                    const float g = agpr_read(acc[i][jj][rr]), u = agpr_read(acc[i][jj + 2][rr]);
                    if (row < M && col < H)
                        st(p.C, p.c_dtype, (size_t)row * H + col, epilogue(g + cb[jj], p.epilogue) * (u + cb[jj + 2]));
                });
                __builtin_amdgcn_sched_barrier(0);
            });
        });
    } else {
        const uint32_t N = p.N, col0 = tn * 256 + wn * 128 + fr;
        static_for<4>([&](auto I) __attribute__((always_inline)) {
            static_for<4>([&](auto J) __attribute__((always_inline)) {
                constexpr int i = I, j = J;
                const uint32_t col = col0 + j * 32;
                static_for<16>([&](auto R) __attribute__((always_inline)) {
                    constexpr int rr = R;
                    const uint32_t row = row0 + i * 32 + (rr % 4) + 8 * (rr / 4);
                    const float a = agpr_read(acc[i][j][rr]);
                    if (row < M && col < N) {
                        const size_t o = (size_t)row * N + col;
                        // a bias other than one [N] row: read per element
                        const float bb = (p.bias && p.bias_repeat != N)
                            ? ld(p.bias, p.bias_dtype, p.bias_repeat ? o % p.bias_repeat : o) : cb[j];
                        const float res = p.residual
                            ? ld(p.residual, p.residual_dtype, p.residual_repeat ? o % p.residual_repeat : o) : 0.f;
                        st(p.C, p.c_dtype, o, finish(a + bb, res, p.epilogue, p.residual_order, p.scalar_scale));
                    }
                });
                __builtin_amdgcn_sched_barrier(0);
            });
        });
    }
}

template <bool GATED>
__device__ __forceinline__ void tile_store(const GemmParams& p, float16v (&acc)[4][4], const float (&cb)[4],
                                           uint32_t tm, uint32_t tn, int wm, int wn, int fr, int fk)
{
    __builtin_amdgcn_sched_barrier(0);
    // Every accumulator passes through an (empty) asm first, so no MFMA can
    // be moved past this point into the epilogue's blocks; the s_nops then
    // give the last MFMA its result-to-read distance.
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) asm volatile("" : "+a"(acc[i][j]));
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");   // MFMA result -> VALU read distance
    const bool cols_in = GATED ? tn * 128 + 128 <= p.H : tn * 256 + 256 <= p.N;
    const bool plain = GATED || (!p.residual && (!p.bias || p.bias_repeat == p.N));   // cb holds the bias
    if (cols_in && plain && p.c_dtype == DT_F32) {
        switch (p.epilogue) {
        case 4: tile_store_fast<GATED, 4>(p, acc, cb, tm, tn, wm, wn, fr, fk); break;   // SiLU
        case 3: tile_store_fast<GATED, 3>(p, acc, cb, tm, tn, wm, wn, fr, fk); break;   // GELU-tanh
        case 0: tile_store_fast<GATED, 0>(p, acc, cb, tm, tn, wm, wn, fr, fk); break;
        default: tile_store_fast<GATED, 6>(p, acc, cb, tm, tn, wm, wn, fr, fk); break;
        }
    } else {
        tile_store_any<GATED>(p, acc, cb, tm, tn, wm, wn, fr, fk);
    }
}

}   // namespace vai_dev
