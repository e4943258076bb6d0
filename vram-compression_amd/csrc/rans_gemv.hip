// Fused rANS decode + batch-1 GEMV for entropy-coded weight codes, written
// for MI355X (gfx950, CDNA4, wave64).  The stream format is the "w64" layout
// documented in include/vramc_rans.h.
//
// Kernel shape (one workgroup = W wavefronts = W tiles of one tile row):
//   1. the 4096-slot symbol table sits in LDS as {freq | code<<24, slot-cum}
//      pairs, so one ds_read_b64 yields both rANS operands and the signed
//      code (the reference keeps sym|freq<<8|bias<<20 and extracts the
//      fields with three more ALU ops per symbol, rans_gemv.cu:33-36).  That
//      32 KB image is built once on the host (rans_table_lds) and copied
//      into LDS with direct global->LDS loads, no registers and no ALU;
//   2. each wavefront copies its tile's compressed block into LDS the same
//      way, 16 bytes per lane, issued together with the table copy;
//   3. each state reads its renormalisation words straight from the staged
//      block at its own offset (a per-state LDS byte address that advances
//      by 2 on each refill);
//   4. each lane runs S independent rANS states; per column step a lane
//      loads x[c]*step[c] once (the waterfilling fold happens here, one block
//      of column steps ahead of use) and reuses it for the R rows of the tile;
//   5. each wave adds its tile's escapes from the side table (into the
//      accumulators before the reduction, or for 35-row tiles into the
//      reduced sums with LDS float adds); row sums are reduced across the 64
//      lanes with a transpose-reduce (permlane swaps and DPP) and across the
//      W waves through LDS in a fixed order, and y is written.  When one
//      workgroup does not cover all column tiles, partial sums go to a
//      workspace and the last workgroup of the tile row adds them up in a
//      fixed order (no atomics on y, no memset, deterministic).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdint>
#include <mutex>
#include <type_traits>

#include "../../include/vramc_rans.h"

namespace {

constexpr uint32_t kProbM = 4096;
constexpr uint32_t kRansL = 1u << 16;
constexpr int kMaxWaves = 8;
// Waves of a workgroup that takes two tile rows (up to five column tiles per
// row); its launch bound allows three waves per SIMD.
constexpr int kMaxWavesRows2 = 10;
// Waves of a decode workgroup (tiles are taken linearly, any count works).
constexpr int kMaxDecodeWaves = 10;

// Table entry in LDS, in one of two layouts:
//   - 8 bytes {freq | code<<24, slot - cum} (T4 = false): one mad consumes
//     both words and the code is the sign-extended top byte;
//   - 4 bytes freq | (slot - cum)<<12 | code<<24 (T4 = true): half the LDS
//     and half the bytes per random table read, for two more VALU
//     instructions per symbol (a mask and a field extract, one of them on
//     the state's dependency chain).  It pays on batch-1 launches with more
//     workgroups than the chip holds at once: the 16 KB saved per
//     workgroup lets more of them share a CU.
template <bool T4>
using TabEntry = std::conditional_t<T4, uint32_t, uint2>;

// Largest batch a GEMV kernel is compiled for with tiles of R rows: 8 for
// tiles of at most 8 rows (one state per lane only), 4 otherwise.
constexpr int gemv_max_batch(int R) { return R <= 8 ? 8 : 4; }

// LDS: the expanded table and the reduction scratch are static __shared__
// arrays (their offsets are compile-time constants, so table addressing
// needs no base add); the per-wave regions are dynamic.  The GEMV's
// reduction scratch holds R*B floats per wave: the host reserves it for the
// largest batch compiled for R and the largest (two-row) workgroup, plus the
// 16-byte arrival flag.
constexpr int gemv_static_lds(int R, bool t4 = false) {
    return (t4 ? 4 : 8) * (int)kProbM + 4 * kMaxWavesRows2 * R * gemv_max_batch(R) + 16;
}
constexpr int kDecodeStaticLds = (int)sizeof(TabEntry<false>) * (int)kProbM;
constexpr int kLdsMax = 160 * 1024;
constexpr int kBufWord3 = 0x00020000;  // buffer resource word 3 for gfx9 raw loads

// 32-bit LDS addresses (address space 3), so a word read is one ds_read with
// no base arithmetic.
using lds_cu16 = const __attribute__((address_space(3))) uint16_t;
using lds_void = __attribute__((address_space(3))) void;
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
__device__ __forceinline__ uint32_t lds_read_u16(uint32_t a) {
    return *(lds_cu16*)(uintptr_t)a;
}

// Per-wave LDS region, in 16-bit words: the staged tile block plus one
// read-ahead word past its end.
struct WaveLayout {
    int raw_words;   // multiple of 8
    int wave_words;  // = raw_words
};

// Per-matrix arguments of a GEMV launch.  A grouped launch runs up to
// kMaxGroup matrices that share x (same cols, tile height, states per lane
// and waves per workgroup) in one grid; matrix i owns the workgroups from
// wg_begin[i] up to the next matrix's.
constexpr int kMaxGroup = 4;
struct MatArgs {
    const uint16_t* words;
    const uint32_t* tile_off;
    const uint8_t* slen;        // length delta | state exponent << 4
    const uint32_t* tile_meta;  // length base | blob words << 16
    const uint4* table_lds;  // 2048 x 16 B LDS image of the table
    const int32_t* esc_tileptr;
    const uint16_t* esc_pos;  // tile-local index c*R + r
    const int16_t* esc_val;
    const float* step;
    float* y;
    int rows, C, ncb;
    int has_esc;    // 0: the side table is empty
    int raw_words;  // LDS words of this matrix's staged block (largest block + 8)
};

struct GemvArgs {
    // first workgroup of matrix i; INT_MAX for unused slots, so the matrix
    // of a workgroup is the number of slots 1.. whose start it has reached
    int wg_begin[kMaxGroup];
    const void* x;
    float* partial;      // [ngroups][B][rows] (one matrix only)
    uint32_t* counters;  // [rows/R]
    int cols, ngroups;
    int W;           // waves per workgroup (= blockDim.x / 64, as a kernel argument)
    int nb;          // x/y rows of this launch, 1..B: a batch-4 kernel also runs a
                     // remainder of 2 or 3 (its other rows re-read the last x row
                     // and store nothing)
    int wave_words;  // per-wave LDS stride (the largest raw_words of the group)
    MatArgs mat[kMaxGroup];
};

struct DecodeArgs {
    const uint16_t* words;
    const uint32_t* tile_off;
    const uint8_t* slen;
    const uint32_t* tile_meta;
    const uint4* table_lds;
    const int32_t* esc_tileptr;
    const uint16_t* esc_pos;  // tile-local index c*R + r
    const int16_t* esc_val;
    const float* step;
    void* out;
    int rows, cols, C, ncb, ntiles;
    int W;        // waves per workgroup
    int has_esc;  // 0: the side table is empty
    WaveLayout L;
};

// freq*(st>>12) + bias (rans_gemv.cu:34): freq < 2^12 and st>>12 < 2^20
// both fit the 24-bit multiplier, whose operand ignores the code byte.
__device__ __forceinline__ uint32_t entry_next_state(uint2 e, uint32_t st) {
    return __umul24(e.x, st >> 12) + e.y;
}

__device__ __forceinline__ int32_t entry_code(uint2 e) { return (int32_t)e.x >> 24; }

// The 4-byte entry: freq is masked out (the multiplier would take the bias
// bits above it) and the bias extracted from bits 12..23.
__device__ __forceinline__ uint32_t entry_next_state(uint32_t e, uint32_t st) {
    return __umul24(e & 0xFFFu, st >> 12) + __builtin_amdgcn_ubfe(e, 12, 12);
}

__device__ __forceinline__ int32_t entry_code(uint32_t e) { return (int32_t)e >> 24; }

// Direct global->LDS copy (global_load_lds_dwordx4): lane i's 16 bytes land
// at the wave-uniform LDS address base + 16*i.  The copy is complete when
// the wave's vector-memory counter has drained (wait_vm).
__device__ __forceinline__ void copy16_to_lds(const uint4* src_lane, void* lds_wave_base) {
    __builtin_amdgcn_global_load_lds(src_lane, (lds_void*)lds_wave_base, 16, 0, 0);
}

// s_waitcnt vmcnt(0) (expcnt and lgkmcnt left at their maxima), as a builtin
// so the compiler's own wait tracking knows every vector load is complete.
__device__ __forceinline__ void wait_vm() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// The table image (32 KB of 8-byte or 16 KB of 4-byte entries, laid out as
// in LDS): chunks of 64 x 16 bytes, wave w of W copying chunks w, w+W, ...
// Issued after the tile block's copy: the table comes from L2 (every
// workgroup reads it), the block from HBM, so the block's copy is the one
// to start first.
template <class E>
__device__ __forceinline__ void stage_table(E* tab, const uint4* __restrict__ img, int wave, int W,
                                            int lane) {
    constexpr int nchunks = (int)(sizeof(E) * kProbM / 1024);
    for (int c = wave; c < nchunks; c += W)
        copy16_to_lds(img + c * 64 + lane, reinterpret_cast<uint4*>(tab) + c * 64);
}

// Extent of tile t's block: tile_off[t], tile_off[t+1] (loaded by every
// lane; the wave-uniform values are taken by tile_extent, as late as
// possible, so the loads issued in between are not waited for).
struct TileOff {
    uint32_t lo, hi;
};
__device__ __forceinline__ TileOff load_tile_off(const uint32_t* __restrict__ tile_off, int t) {
    return {tile_off[t], tile_off[t + 1]};
}

// Start (in words) and length (in 16-byte units, at most the region) of the
// block, as scalars; n16 is 0 for an inactive wave.
__device__ __forceinline__ void tile_extent(TileOff to, bool active, int raw_words, uint32_t& o0,
                                            uint32_t& n16) {
    uint32_t nw = to.hi - to.lo;
    if (nw > (uint32_t)raw_words) nw = (uint32_t)raw_words;
    o0 = __builtin_amdgcn_readfirstlane(to.lo);
    n16 = active ? __builtin_amdgcn_readfirstlane(nw >> 3) : 0u;
}

// The wave's tile block (n16 x 16 bytes at words + 8*o16) into its LDS region.
__device__ __forceinline__ void stage_tile(uint16_t* raw, const uint16_t* __restrict__ words,
                                           uint32_t o0, uint32_t n16, int lane) {
    const uint4* src = reinterpret_cast<const uint4*>(words + o0);
    for (uint32_t c = 0; c < n16; c += 64)
        if (c + lane < n16) copy16_to_lds(src + c + lane, reinterpret_cast<uint4*>(raw) + c);
}

__device__ __forceinline__ uint32_t load_x_bits(const void* x, int64_t i, bool bf16) {
    if (bf16) return reinterpret_cast<const uint16_t*>(x)[i];
    return reinterpret_cast<const uint32_t*>(x)[i];
}

__device__ __forceinline__ float bits_to_x(uint32_t v, bool bf16) {
    return __uint_as_float(bf16 ? v << 16 : v);
}

template <typename T>
__device__ __forceinline__ T raw_load(__amdgpu_buffer_rsrc_t r, int off) {
    if constexpr (std::is_same_v<T, __bf16>)
        return __builtin_bit_cast(__bf16, __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0));
    else
        return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}

__device__ __forceinline__ float raw_to_x(__bf16 v) { return (float)v; }
__device__ __forceinline__ float raw_to_x(uint32_t v) { return __uint_as_float(v); }

__device__ __forceinline__ float load_x(const void* x, int64_t i, bool bf16) {
    return bits_to_x(load_x_bits(x, i, bf16), bf16);
}

// v from lane (dpp CTRL) for the rows in ROWS; 0 in the other rows.
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWS, 0xF, false));
}

// Sum over the 64 lanes with DPP moves (no LDS round trips); the total is
// valid in lane 63.  Fixed order, so the result is deterministic.
__device__ __forceinline__ float wave_sum63(float v) {
    v += dpp<0xB1>(v);        // quad_perm [1,0,3,2]
    v += dpp<0x4E>(v);        // quad_perm [2,3,0,1]: quad sums
    v += dpp<0x141>(v);       // row_half_mirror: sums of 8
    v += dpp<0x140>(v);       // row_mirror: row (16-lane) sums
    v += dpp<0x142, 0xA>(v);  // row_bcast:15 into rows 1, 3
    v += dpp<0x143, 0xC>(v);  // row_bcast:31 into rows 2, 3
    return v;
}

// Sums each of N values (a power of two up to 64) over the 64 lanes with
// about 2.2*N instructions instead of 6*N.  Stage j (j = 0..5) pairs the
// lanes that differ in lane-id bit 5-j.  While a lane holds n > 1 values it
// keeps the half selected by that bit and adds its partner's copy of the
// same half, so the value count halves; once n = 1 a stage is a plain pair
// sum.  Partners: v_permlane32_swap / v_permlane16_swap exchange the halves
// directly for bits 5 and 4; DPP row_mirror, row_half_mirror and quad_perm
// reach them for bits 3..0 (a mirror pairs lanes differing in that bit, and
// lanes that share the bits already summed hold disjoint lane sets).  Every
// lane ends with the complete total of value index lane >> (6 - log2 N).
template <int J, int N>
__device__ __forceinline__ void wave_transpose_stage(float* w, int lane) {
    if constexpr (J < 6) {
        constexpr int bit = 5 - J;
        constexpr int CTRL = J == 2 ? 0x140 : J == 3 ? 0x141 : J == 4 ? 0x4E : 0xB1;
        constexpr int h = N > 1 ? N / 2 : 1;
        const bool hi = (lane >> bit) & 1;
#pragma unroll
        for (int i = 0; i < h; i++) {
            const float a = w[i], b = N > 1 ? w[i + h] : w[i];
            if constexpr (J == 0) {
                const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b),
                                                                false, false);
                w[i] = __uint_as_float(p[0]) + __uint_as_float(p[1]);
            } else if constexpr (J == 1) {
                const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b),
                                                                false, false);
                w[i] = __uint_as_float(p[0]) + __uint_as_float(p[1]);
            } else if constexpr (N > 1) {
                w[i] = (hi ? b : a) + dpp<CTRL>(hi ? a : b);
            } else {
                w[i] = a + dpp<CTRL>(a);
            }
        }
        wave_transpose_stage<J + 1, h>(w, lane);
    }
}

template <int N>
__device__ __forceinline__ float wave_transpose_sum(float (&v)[N], int lane) {
    static_assert(N >= 1 && N <= 64 && (N & (N - 1)) == 0, "N must be a power of two <= 64");
    wave_transpose_stage<0, N>(v, lane);
    return v[0];
}

constexpr int ilog2(int n) { return n <= 1 ? 0 : 1 + ilog2(n / 2); }

// Sums each of the N values w[OFF..OFF+N) over the 64 lanes into
// out[OFF..OFF+N), for any N: power-of-two chunks of at most 64 values,
// largest first (35 = 32 + 2 + 1), each through wave_transpose_sum.
template <int OFF, int N, int NT>
__device__ __forceinline__ void transpose_sum_store(const float (&w)[NT], float* out, int lane) {
    if constexpr (N > 0) {
        constexpr int C = N >= 64 ? 64 : 1 << ilog2(N);
        float v[C];
#pragma unroll
        for (int i = 0; i < C; i++) v[i] = w[OFF + i];
        const float t = wave_transpose_sum<C>(v, lane);
        constexpr int sh = 6 - ilog2(C);
        if ((lane & ((1 << sh) - 1)) == 0) out[OFF + (lane >> sh)] = t;
        transpose_sum_store<OFF + C, N - C, NT>(w, out, lane);
    }
}

// Inclusive prefix sum over the 64 lanes: within each 16-lane row with
// row_shr 1, 2, 4, 8 (a lane without a source in its row adds 0), then the
// row totals carried into the rows above with row_bcast 15 and 31.
__device__ __forceinline__ uint32_t wave_scan(uint32_t v) {
    v += __builtin_amdgcn_update_dpp(0u, v, 0x111, 0xF, 0xF, false);  // row_shr:1
    v += __builtin_amdgcn_update_dpp(0u, v, 0x112, 0xF, 0xF, false);  // row_shr:2
    v += __builtin_amdgcn_update_dpp(0u, v, 0x114, 0xF, 0xF, false);  // row_shr:4
    v += __builtin_amdgcn_update_dpp(0u, v, 0x118, 0xF, 0xF, false);  // row_shr:8
    v += __builtin_amdgcn_update_dpp(0u, v, 0x142, 0xA, 0xF, false);  // row_bcast:15 to rows 1, 3
    v += __builtin_amdgcn_update_dpp(0u, v, 0x143, 0xC, 0xF, false);  // row_bcast:31 to rows 2, 3
    return v;
}

// Where each of the lane's S states lives in the tile block, from its
// length byte lb (length - base | exponent << 4) and the tile's meta word
// (base | blob words << 16): off, the word offset of its stream (the
// streams follow the blob in state order, j = s*64 + lane), and bit, the
// bit offset of its initial state's mantissa in the blob (16 + e bits per
// state, in state order).  Both sums go through one scan, packed in the two
// halves of a word (a wave's lengths stay below 2^16 words and its
// mantissas below 2^11 bits).
template <int S>
__device__ __forceinline__ void stream_layout(const uint32_t (&lb)[S], uint32_t meta,
                                              uint32_t (&off)[S], uint32_t (&bit)[S]) {
    const uint32_t base = meta & 0xFFu;
    uint32_t ocarry = meta >> 16, bcarry = 0;
#pragma unroll
    for (int s = 0; s < S; s++) {
        const uint32_t v = (base + (lb[s] & 15u)) | (16u + (lb[s] >> 4)) << 16;
        const uint32_t inc = wave_scan(v);
        const uint32_t ex = inc - v;
        off[s] = ocarry + (ex & 0xFFFFu);
        bit[s] = bcarry + (ex >> 16);
        const uint32_t tot = __builtin_amdgcn_readlane(inc, 63);
        ocarry += tot & 0xFFFFu;
        bcarry += tot >> 16;
    }
}

// A state's initial value from the staged blob: the 16 + e bits at bit
// offset `bit` below an implicit leading one.
__device__ __forceinline__ uint32_t initial_state(const uint16_t* raw, uint32_t bit, uint32_t lb) {
    const uint32_t* r32 = reinterpret_cast<const uint32_t*>(raw);
    const uint32_t lo = r32[bit >> 5], hi = r32[(bit >> 5) + 1];
    const uint32_t nb = 16u + (lb >> 4);
    return __builtin_amdgcn_ubfe(__builtin_amdgcn_alignbit(hi, lo, bit & 31u), 0, nb) | (1u << nb);
}

// Per-lane decoder state of S interleaved rANS states, with the table entry
// of each state's next symbol already read (software pipelined: the read for
// symbol i+1 is issued before the GEMV work of symbol i).
template <int S, class E>
struct Lanes {
    uint32_t st[S];  // rANS states
    uint32_t a[S];   // LDS byte address of the next unread word of each state
    uint32_t w[S];   // that word (read ahead)
    E e[S];          // table entry for the next symbol of each state
};

// Staged-block setup: each state's read pointer, its first word and the
// table entry of its first symbol.  Call after the staging barrier.
template <int S, class E>
__device__ __forceinline__ void init_lanes(Lanes<S, E>& L, const E* tab, const uint16_t* raw,
                                           const uint32_t (&st0)[S], const uint32_t (&off0)[S]) {
#pragma unroll
    for (int s = 0; s < S; s++) {
        L.st[s] = st0[s];
        L.a[s] = lds_addr(raw + off0[s]);
        L.w[s] = lds_read_u16(L.a[s]);
        L.e[s] = tab[L.st[s] & (kProbM - 1)];
    }
}

// One rANS decode step with the reference arithmetic (rans_gemv.cu:32-37):
// st = freq*(st>>12) + bias from the entry e = tab[st & 4095]; renormalise
// with the next stream word when st < 2^16; return the symbol's code.  The
// entry for the following symbol is read as soon as the new state exists,
// before the code conversion and the word-pointer update, so those overlap
// the LDS latency instead of sitting on the state's dependency chain.
//
// The next word w is always read ahead.  REFILL=false: every lane re-reads
// it each step (no divergence, the cheapest step when LDS is not the
// bottleneck).  REFILL=true: only the lanes that just consumed their word
// fetch the next one (an EXEC-masked read, about 1 lane in 5 at 3 bits per
// symbol), which cuts LDS bank traffic where many waves share the CU.
template <bool REFILL, class E>
__device__ __forceinline__ int32_t rans_step(uint32_t& st, uint32_t& a, uint32_t& w, E& e,
                                             const E* tab) {
    const E cur = e;
    const uint32_t ns = entry_next_state(cur, st);
    const bool need = ns < kRansL;
    st = need ? ((ns << 16) | w) : ns;
    e = tab[st & (kProbM - 1)];
    if (REFILL) {
        if (need) {
            a += 2u;
            w = lds_read_u16(a);
        }
    } else {
        a += need ? 2u : 0u;
        w = lds_read_u16(a);
    }
    return entry_code(cur);
}

// Tile row and tile column of a side-table position c*R + r (R is a
// compile-time constant, so the division is a multiply and shift).
template <int R>
__device__ __forceinline__ int esc_row(int pos) { return (int)((uint32_t)pos % (uint32_t)R); }
template <int R>
__device__ __forceinline__ uint32_t esc_tcol(int pos) { return (uint32_t)pos / (uint32_t)R; }

// Adds an escape entry at tile row re to the lane's accumulators; v[b] is
// value*step*x[b] (0 for a lane without an entry).  A 0/1 weight per row and
// one FMA per (row, batch): 2R + RB instructions rather than R + 2RB for a
// select and an add.
template <int R, int B>
__device__ __forceinline__ void add_escape(float (&acc)[R][B], int re, const float (&v)[B]) {
#pragma unroll
    for (int r = 0; r < R; r++) {
        const float m = re == r ? 1.f : 0.f;
#pragma unroll
        for (int b = 0; b < B; b++) acc[r][b] = fmaf(m, v[b], acc[r][b]);
    }
}

// Adds v to a float in LDS (ds_add_f32; no value returned).
__device__ __forceinline__ void lds_add(float* p, float v) {
    __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Escapes of 35-row tiles go to the reduced row sums in LDS with one float
// add per lane and batch row instead of 2R + RB VALU instructions per chunk.
// That pays while the LDS is otherwise idle: R = 35 tiles run two waves per
// SIMD (8960 x 1536).  With four waves per SIMD (large matrices, 16-row
// tiles) the atomics, serialised on the CU's one LDS, cost more than the
// FMAs (25600x5120 with 1% escapes: +6% at batch 1, +38% at batch 4), so
// 20-row tiles (made for large matrices) keep the FMAs.
template <int R>
constexpr bool kEscapesInLds = R == 35;

// GROUP: a grouped launch (several matrices, slot found per workgroup);
// otherwise slot 0 only, read at fixed kernel-argument offsets.  T4: the
// 4-byte table entries (the slot's table_lds then points at that image).
// ROWS2: each workgroup takes two adjacent tile rows, W/2 waves each, so
// one table copy serves twice the waves (single pass over the columns
// only: no split-K).
// Waves per SIMD the register allocation must allow: 4 for the kernels
// with 64 or more accumulators beside the decode state (the batch-4 kernel
// on 20-row tiles and the batch-8 kernel on 8-row tiles), which otherwise
// take 130 VGPRs and 3 waves per SIMD (25600x5120 at batch 4: 86.5 us; at
// 128 VGPRs, one register spilled outside the decode loop, 61.8 us); 1 (no
// constraint) elsewhere.
template <int R, int B>
constexpr int kMinWavesPerEu = ((R == 20 && B == 4) || (R == 8 && B == 8)) ? 4 : 1;

template <int R, int S, int B, bool XBF16, bool REFILL, bool GROUP, bool T4, bool ROWS2>
__global__ void __launch_bounds__(64 * (ROWS2 ? kMaxWavesRows2 : kMaxWaves))
    __attribute__((amdgpu_waves_per_eu(kMinWavesPerEu<R, B>)))
    rans_w64_gemv_kernel(GemvArgs a) {
    __shared__ __align__(16) TabEntry<T4> tab[kProbM];
    __shared__ float red[(ROWS2 ? kMaxWavesRows2 : kMaxWaves) * R * B];
    __shared__ int flag[4];
    extern __shared__ __align__(16) uint16_t dyn[];
    constexpr int nst = 64 * S;
    const int W = a.W;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar tile math
    const int lane = threadIdx.x & 63;
    uint16_t* raw = dyn + (size_t)wave * a.wave_words;

    // This workgroup's matrix.  A grouped launch reads its slot through an
    // index (one more dependent scalar load); a single-matrix launch reads
    // slot 0 at fixed offsets, fetched with the rest of the arguments.
    int mi = 0;
    if constexpr (GROUP) {
#pragma unroll
        for (int i = 1; i < kMaxGroup; i++) mi += (int)blockIdx.x >= a.wg_begin[i] ? 1 : 0;
    }
    const MatArgs& m = a.mat[GROUP ? mi : 0];
    // Every kernel argument the prologue needs, fetched in one scalar batch
    // (otherwise each is loaded, and waited for, at its first use).
    asm volatile("" ::"s"(m.tile_off), "s"(m.tile_meta), "s"(m.slen), "s"(m.table_lds),
                 "s"(m.words), "s"(a.x), "s"(m.step), "s"(m.esc_tileptr), "s"(m.esc_pos),
                 "s"(m.esc_val), "s"(m.C), "s"(a.cols),
                 "s"(m.raw_words), "s"(a.W), "s"(m.ncb), "s"(a.ngroups), "s"(a.nb));
    const int bid = (int)blockIdx.x - (GROUP ? a.wg_begin[mi] : 0);
    constexpr int RPW = ROWS2 ? 2 : 1;  // tile rows per workgroup
    const int Wt = ROWS2 ? W / 2 : W;   // waves per tile row
    const int rsub = ROWS2 ? (wave >= Wt ? 1 : 0) : 0;
    const int rb0 = (bid / a.ngroups) * RPW;
    const int rb = rb0 + rsub;
    const int g = bid - (bid / a.ngroups) * a.ngroups;
    const int cb = g * Wt + (wave - rsub * Wt);  // Wt divides ncb: every wave has a tile
    const int t = rb * m.ncb + cb;

    // Everything the wave needs from memory before decoding is requested in
    // one batch: initial states, stream offsets, the first block of x and
    // step, the table and the tile block.
    const int nk = m.C / nst;
    const int colbase = cb * m.C + lane;
    // The tile extent is loaded first: the block copy waits for it, and
    // loads complete in order, so nothing issued after it delays that copy.
    const TileOff to = load_tile_off(m.tile_off, t);
    // This tile's range of the escape side table (lanes 0, 1), also needed early.
    const int tp = m.esc_tileptr[t + min(lane, 1)];
    asm volatile("" ::: "memory");  // keep these two loads first
    // The kernels for launches that put several workgroups on a CU (the
    // 4-byte table entries, chosen where the grid exceeds what the chip
    // holds, tiles of 20 or more rows, and the batch kernels outside paired
    // rows) start the table copy while the tile extent is on its way; the
    // others request the block copy first, so that it does not queue behind
    // the table.
    constexpr bool kTableFirst = T4 || R >= 20 || (B >= 4 && !ROWS2);
    if constexpr (kTableFirst) stage_table(tab, m.table_lds, wave, W, lane);
    const uint32_t tmv = m.tile_meta[t];
    uint32_t len0[S];
#pragma unroll
    for (int s = 0; s < S; s++) len0[s] = m.slen[t * nst + 64 * s + lane];
    // x and step for KU column steps are loaded one block ahead of use, so
    // their latency overlaps the decode of the current block.  They are
    // buffer loads ranged to one x row / the step vector: a block's columns
    // are immediate offsets on one base register, and columns past the end
    // of the matrix (the tail of the last block) read as 0.
    // column steps per prefetch block: 4, or 2 where the prefetch registers
    // would otherwise cost occupancy (S=4, or a batch of 4)
    constexpr int KU = (S >= 4 || B >= 4) ? 2 : 4;
    constexpr int XS = XBF16 ? 2 : 4;
    __amdgpu_buffer_rsrc_t xrs[B];
#pragma unroll
    for (int b = 0; b < B; b++)
        xrs[b] = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint8_t*>(static_cast<const uint8_t*>(a.x)) + (size_t)min(b, a.nb - 1) * a.cols * XS,
            0, a.cols * XS, kBufWord3);
    const __amdgpu_buffer_rsrc_t srs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(m.step), 0, a.cols * 4, kBufWord3);
    // bf16 values kept as __bf16 (an integer register pin would be widened
    // first, at the cost of a mask per value), or f32 bits
    using XRaw = std::conditional_t<XBF16, __bf16, uint32_t>;
    XRaw xr[KU][S][B];
    float sr[KU][S];
    auto load_block = [&](int k0) {
        const int c0 = colbase + 64 * S * k0;
#pragma unroll
        for (int u = 0; u < KU; u++) {
#pragma unroll
            for (int s = 0; s < S; s++) {
                const int c = c0 + 64 * (S * u + s);
                sr[u][s] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(srs, c * 4, 0, 0));
#pragma unroll
                for (int b = 0; b < B; b++)
                    xr[u][s][b] =
                        raw_load<XRaw>(xrs[b], XBF16 ? c * 2 : c * 4);
            }
        }
    };
    load_block(0);
    uint32_t o0, n16;
    tile_extent(to, true, m.raw_words, o0, n16);
    // Each wave adds its own tile's escapes, in chunks of 64 side-table
    // entries.  They run in column order within the tile, so a chunk's x and
    // step gathers fall in a narrow column range (a few cache lines).  The
    // range is read here, before the copies, while the wait for it is exact;
    // the first chunks are requested behind the copies (so waiting for them
    // costs nothing more), and their x and step gathers go out before the
    // decode loop, their values kept raw until after the loop, so that
    // latency overlaps the decode.
    const bool esc = m.has_esc;  // kernel-uniform
    const int e_lo = esc ? __builtin_amdgcn_readlane(tp, 0) : 0;
    const int e_hi = esc ? __builtin_amdgcn_readlane(tp, 1) : 0;
    asm volatile("" ::"s"(e_lo), "s"(e_hi));
    stage_tile(raw, m.words, o0, n16, lane);
    if constexpr (!kTableFirst) stage_table(tab, m.table_lds, wave, W, lane);
    constexpr int P = 2;  // chunks per wave prefetched: 128 escapes per tile
    const int cbase = cb * m.C;
    // tile column of an entry, clamped into the tile so that no side-table
    // content can send a gather outside x or step
    auto esc_col = [&](int pos) { return cbase + (int)min(esc_tcol<R>(pos), (uint32_t)(m.C - 1)); };
    int epos[P], eval[P];
#pragma unroll
    for (int p = 0; p < P; p++) {
        epos[p] = eval[p] = 0;
        if (e_lo + 64 * p < e_hi) {  // wave-uniform
            const int ec = min(e_lo + 64 * p + lane, e_hi - 1);
            epos[p] = m.esc_pos[ec];
            eval[p] = m.esc_val[ec];
        }
    }
    wait_vm();
    __syncthreads();
    float acc[R][B];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int b = 0; b < B; b++) acc[r][b] = 0.f;

    // x*step of the current block, converted at the top of each iteration.
    float xv[KU][S][B];
    auto convert = [&]() {
#pragma unroll
        for (int u = 0; u < KU; u++)
#pragma unroll
            for (int s = 0; s < S; s++) {
                // pin the prefetched registers here so the multiply is not
                // hoisted next to their loads
                asm volatile("" : "+v"(sr[u][s]));
#pragma unroll
                for (int b = 0; b < B; b++) {
                    asm volatile("" : "+v"(xr[u][s][b]));
                    xv[u][s][b] = raw_to_x(xr[u][s][b]) * sr[u][s];
                    // all multiplies here, so the prefetch that follows can
                    // overwrite sr and xr without copies
                    asm volatile("" : "+v"(xv[u][s][b]));
                }
            }
    };
    // Escape gathers: issued in the first iteration behind the prefetch of
    // the second block, so the first wait that can drain them comes a block
    // of decode later.  Unconditional (the tile's first column for a wave
    // without a chunk): no branch, so no register merges that would wait
    // for them early.
    uint32_t exr[P][B], esr[P];
    auto gather = [&]() {
#pragma unroll
        for (int p = 0; p < P; p++) {
            asm volatile("" : "+v"(epos[p]), "+v"(eval[p]));
            const int col = esc_col(epos[p]);
            esr[p] = __float_as_uint(m.step[col]);
#pragma unroll
            for (int b = 0; b < B; b++)
                exr[p][b] = load_x_bits(a.x, (int64_t)min(b, a.nb - 1) * a.cols + col, XBF16);
        }
    };

    {
        Lanes<S, TabEntry<T4>> L;
        uint32_t off0[S], bit0[S], st0[S];
        stream_layout<S>(len0, __builtin_amdgcn_readfirstlane(tmv), off0, bit0);
#pragma unroll
        for (int s = 0; s < S; s++) st0[s] = initial_state(raw, bit0[s], len0[s]);
        init_lanes(L, tab, raw, st0, off0);
        for (int k0 = 0; k0 < nk; k0 += KU) {
            convert();
            // unconditional: past the last block these read columns of the
            // next tile, or 0 past the end of the matrix, and go unused; a
            // conditional prefetch makes the compiler copy the registers
            load_block(k0 + KU);
            if (k0 == 0 && esc) gather();
            // keep the prefetch here: without this the scheduler sinks the
            // loads below the decode and the next block waits on them
            asm volatile("" ::: "memory");
#pragma unroll
            for (int u = 0; u < KU; u++) {
                if (k0 + u >= nk) break;
#pragma unroll
                for (int r = 0; r < R; r++) {
#pragma unroll
                    for (int s = 0; s < S; s++) {
                        const float code =
                            (float)rans_step<REFILL>(L.st[s], L.a[s], L.w[s], L.e[s], tab);
#pragma unroll
                        for (int b = 0; b < B; b++) {
                            acc[r][b] = fmaf(code, xv[u][s][b], acc[r][b]);
                            // with the refill branches the compiler sinks
                            // the conversions and FMAs to the end of the
                            // block, keeping every step's 64-bit table entry
                            // live; consuming the sum here keeps them in place
                            if (REFILL) asm volatile("" : "+v"(acc[r][b]));
                        }
                    }
                }
            }
        }
    }

    if constexpr (!kEscapesInLds<R>) {
        float ev[B];
#pragma unroll
        for (int p = 0; p < P; p++) {
            const int e = e_lo + 64 * p + lane;
            if (e_lo + 64 * p < e_hi) {
                asm volatile("" : "+v"(esr[p]));
#pragma unroll
                for (int b = 0; b < B; b++) asm volatile("" : "+v"(exr[p][b]));
                const float ve = e < e_hi ? (float)eval[p] * __uint_as_float(esr[p]) : 0.f;
#pragma unroll
                for (int b = 0; b < B; b++) ev[b] = ve * bits_to_x(exr[p][b], XBF16);
                add_escape<R, B>(acc, esc_row<R>(epos[p]), ev);
            }
        }
        // further chunks (tiles with more than 64*P escapes)
        for (int e0 = e_lo + 64 * P; e0 < e_hi; e0 += 64) {
            const int e = e0 + lane;
            const int ec = min(e, e_hi - 1);
            const int pos = m.esc_pos[ec];
            const int col = esc_col(pos);
            const float ve = e < e_hi ? (float)m.esc_val[ec] * m.step[col] : 0.f;
#pragma unroll
            for (int b = 0; b < B; b++)
                ev[b] = ve * load_x(a.x, (int64_t)min(b, a.nb - 1) * a.cols + col, XBF16);
            add_escape<R, B>(acc, esc_row<R>(pos), ev);
        }
    }

    // Every (row, batch) sum goes through the transpose-reduce, whatever
    // R*B: its lanes pair in the same order for any value count, so the
    // batch-1, -4 and -8 kernels give bitwise the same sum for a vector, and
    // a batch split into chunks differently (grouped, paired rows, either
    // table layout) gives the same results.
    constexpr int NRB = R * B;
    {
        float w[NRB];
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int b = 0; b < B; b++) w[r * B + b] = acc[r][b];
        transpose_sum_store<0, NRB, NRB>(w, red + wave * NRB, lane);
    }

    // Tall tiles: the escapes added to the wave's reduced sums, each lane
    // with a side-table entry adding value*step*x[b] to its row's slot.  The
    // wave's own stores above come first (a wave's LDS operations complete
    // in order), and lanes of one instruction that share a slot are
    // serialised in a fixed order, so the sums are deterministic.  Rows
    // outside the tile are skipped.
    if constexpr (kEscapesInLds<R>) {
        float* wred = red + wave * NRB;
#pragma unroll
        for (int p = 0; p < P; p++) {
            const int e = e_lo + 64 * p + lane;
            if (e_lo + 64 * p < e_hi) {
                asm volatile("" : "+v"(esr[p]));
#pragma unroll
                for (int b = 0; b < B; b++) asm volatile("" : "+v"(exr[p][b]));
                const int re = esc_row<R>(epos[p]);
                if (e < e_hi && re < R) {
                    const float ve = (float)eval[p] * __uint_as_float(esr[p]);
#pragma unroll
                    for (int b = 0; b < B; b++)
                        lds_add(&wred[re * B + b], ve * bits_to_x(exr[p][b], XBF16));
                }
            }
        }
        // further chunks (tiles with more than 64*P escapes)
        for (int e0 = e_lo + 64 * P; e0 < e_hi; e0 += 64) {
            const int e = e0 + lane;
            const int ec = min(e, e_hi - 1);
            const int pos = m.esc_pos[ec];
            const int re = esc_row<R>(pos);
            const int col = esc_col(pos);
            const float ve = (float)m.esc_val[ec] * m.step[col];
            float xb[B];
#pragma unroll
            for (int b = 0; b < B; b++)
                xb[b] = load_x(a.x, (int64_t)min(b, a.nb - 1) * a.cols + col, XBF16);
            if (e < e_hi && re < R) {
#pragma unroll
                for (int b = 0; b < B; b++) lds_add(&wred[re * B + b], ve * xb[b]);
            }
        }
    }
    __syncthreads();

    // Per (row, batch) totals over the workgroup's waves, entry i = r*B + b.
    // R*B can exceed the workgroup's threads (R = 35 at batch 4).
    const int tid = threadIdx.x;
    const int nthr = 64 * W;
    auto total = [&](int i) {
        float v = 0.f;
        for (int ww = 0; ww < W; ww++) v += red[ww * NRB + i];
        return v;
    };
    if constexpr (ROWS2) {
        // each tile row summed over its own waves, in the same order as a
        // one-row workgroup sums its W waves
        for (int i = tid; i < RPW * NRB; i += nthr) {
            const int rs = i / NRB, ii = i - rs * NRB;
            float v = 0.f;
            for (int ww = 0; ww < Wt; ww++) v += red[(rs * Wt + ww) * NRB + ii];
            const int r = ii / B, b = ii - r * B;
            if (b < a.nb) m.y[(int64_t)b * m.rows + (rb0 + rs) * R + r] = v;
        }
        return;
    }
    if (a.ngroups == 1) {
        for (int i = tid; i < NRB; i += nthr) {
            const int r = i / B, b = i - r * B;
            if (b < a.nb) m.y[(int64_t)b * m.rows + rb * R + r] = total(i);
        }
        return;
    }

    // Split over column groups: publish the partial, count arrivals, and let
    // the last workgroup of this tile row sum the partials in group order.
    // Partials are written with agent-scope atomic stores, which write
    // through the per-XCD L2, and every thread waits for its store to
    // complete before the barrier; the arrival counter is then bumped and
    // the last workgroup reads the partials with agent-scope (coherent)
    // loads.  This avoids release/acquire fences, which on this chip write
    // back or invalidate the whole L2 of the XCD.
    for (int i = tid; i < NRB; i += nthr) {
        const int r = i / B, b = i - r * B;
        __hip_atomic_store(&a.partial[((int64_t)g * B + b) * m.rows + rb * R + r], total(i),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
        const uint32_t old = __hip_atomic_fetch_add(&a.counters[rb], 1u, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT);
        *flag = old == (uint32_t)(a.ngroups - 1);
    }
    __syncthreads();
    if (*flag) {
        for (int i = tid; i < NRB; i += nthr) {
            const int r = i / B, b = i - r * B;
            float s = 0.f;
            for (int gg = 0; gg < a.ngroups; gg++)
                s += __hip_atomic_load(&a.partial[((int64_t)gg * B + b) * m.rows + rb * R + r],
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (b < a.nb) m.y[(int64_t)b * m.rows + rb * R + r] = s;
        }
        if (tid == 0)
            __hip_atomic_store(&a.counters[rb], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// bf16 of f, round to nearest even (gfx950's v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint16_t to_bf16(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

// Decode only.  MODE 0 writes int32 codes, MODE 1 writes bf16(code*step[c]).
// One wave per tile, the staging and decode step of the GEMV.  Output goes
// through one buffer resource over the tile row's R output rows: a store's
// row is its scalar offset, its column step an immediate.  After its own
// stores have completed, each wave overwrites the escape positions of its
// tile (decoded as 0) with their side-table values, so no second launch.
template <int R, int S, int MODE>
__global__ void __launch_bounds__(64 * kMaxDecodeWaves) rans_w64_decode_kernel(DecodeArgs a) {
    __shared__ __align__(16) TabEntry<false> tab[kProbM];
    extern __shared__ __align__(16) uint16_t dyn[];
    constexpr int nst = 64 * S;
    constexpr int ESZ = MODE == 0 ? 4 : 2;
    constexpr int KU = S >= 4 ? 2 : 4;
    const int W = a.W;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar tile math
    const int lane = threadIdx.x & 63;
    uint16_t* raw = dyn + (size_t)wave * a.L.wave_words;
    const int t = blockIdx.x * W + wave;
    const bool active = t < a.ntiles;
    const int tc = active ? t : a.ntiles - 1;
    const int rb = tc / a.ncb, cb = tc - rb * a.ncb;
    asm volatile("" ::"s"(a.tile_off), "s"(a.tile_meta), "s"(a.slen), "s"(a.table_lds),
                 "s"(a.words), "s"(a.step), "s"(a.esc_tileptr), "s"(a.out), "s"(a.C),
                 "s"(a.cols), "s"(a.L.raw_words), "s"(a.W), "s"(a.ncb), "s"(a.ntiles));

    const TileOff to = load_tile_off(a.tile_off, tc);
    const int tp = a.esc_tileptr[tc + min(lane, 1)];
    asm volatile("" ::: "memory");  // keep these two loads first
    const uint32_t tmv = a.tile_meta[tc];
    uint32_t len0[S];
#pragma unroll
    for (int s = 0; s < S; s++) len0[s] = a.slen[tc * nst + 64 * s + lane];
    const int nk = a.C / nst;
    const int colbase = cb * a.C + lane;
    const __amdgpu_buffer_rsrc_t srs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(a.step), 0, a.cols * 4, kBufWord3);
    float sr[KU][S];
    auto load_steps = [&](int k0) {
        const int c0 = colbase + 64 * S * k0;
#pragma unroll
        for (int u = 0; u < KU; u++)
#pragma unroll
            for (int s = 0; s < S; s++)
                sr[u][s] = __uint_as_float(
                    __builtin_amdgcn_raw_buffer_load_b32(srs, (c0 + 64 * (S * u + s)) * 4, 0, 0));
    };
    if (MODE == 1) load_steps(0);
    uint32_t o0, n16;
    tile_extent(to, active, a.L.raw_words, o0, n16);
    stage_tile(raw, a.words, o0, n16, lane);
    stage_table(tab, a.table_lds, wave, W, lane);
    wait_vm();
    __syncthreads();
    if (!active) return;

    uint8_t* obase = static_cast<uint8_t*>(a.out) + (size_t)rb * R * a.cols * ESZ;
    const __amdgpu_buffer_rsrc_t ors =
        __builtin_amdgcn_make_buffer_rsrc(obase, 0, R * a.cols * ESZ, kBufWord3);
    Lanes<S, TabEntry<false>> L;
    uint32_t off0[S], bit0[S], st0[S];
    stream_layout<S>(len0, __builtin_amdgcn_readfirstlane(tmv), off0, bit0);
#pragma unroll
    for (int s = 0; s < S; s++) st0[s] = initial_state(raw, bit0[s], len0[s]);
    init_lanes(L, tab, raw, st0, off0);
    // One block of nu <= KU column steps.  The loop below runs whole blocks
    // only (nu = KU, no early exit): exits after 1, 2 or 3 steps' stores
    // would meet at the loop latch, and the compiler would then wait there
    // for the stores of the longest path.  A partial last block follows it.
    auto run_block = [&](int k0, int nu) {
        float sv[KU][S];
        if (MODE == 1) {
#pragma unroll
            for (int u = 0; u < KU; u++)
#pragma unroll
                for (int s = 0; s < S; s++) {
                    asm volatile("" : "+v"(sr[u][s]));
                    sv[u][s] = sr[u][s];
                }
            // unconditional: past the last block these read columns of the
            // next tile, or 0 past the end of the matrix, and go unused.  A
            // conditional prefetch merges two wait states at the join, and
            // the compiler then waits for this block's stores as well
            // (vmcnt counts stores too), once per block
            load_steps(k0 + KU);
            asm volatile("" ::: "memory");
        }
        const int vb = (colbase + 64 * S * k0) * ESZ;
#pragma unroll
        for (int u = 0; u < KU; u++) {
            if (u >= nu) break;
#pragma unroll
            for (int r = 0; r < R; r++) {
#pragma unroll
                for (int s = 0; s < S; s++) {
                    // symbol order within a state is k-major, r-minor, as in the GEMV
                    const int32_t code = rans_step<(R >= 8)>(L.st[s], L.a[s], L.w[s], L.e[s], tab);
                    const int vo = vb + 64 * (S * u + s) * ESZ;
                    if (MODE == 0)
                        __builtin_amdgcn_raw_buffer_store_b32(code, ors, vo, r * a.cols * 4, 0);
                    else
                        __builtin_amdgcn_raw_buffer_store_b16(to_bf16((float)code * sv[u][s]), ors,
                                                              vo, r * a.cols * 2, 0);
                }
            }
        }
    };
    const int nk_full = nk - nk % KU;
    for (int k0 = 0; k0 < nk_full; k0 += KU) run_block(k0, KU);
    if (nk_full < nk) run_block(nk_full, nk - nk_full);

    // Escapes of this tile: its own side-table entries, written over the 0
    // each escape position was decoded as.  The wave's own stores complete
    // first, so the value lands after that 0.  Positions are clamped into
    // the tile, so no side-table content can address outside the output.
    if (!a.has_esc) return;
    wait_vm();
    const int e_lo = __builtin_amdgcn_readlane(tp, 0), e_hi = __builtin_amdgcn_readlane(tp, 1);
    const int cbase = cb * a.C;
    for (int e = e_lo + lane; e < e_hi; e += 64) {
        const int pos = a.esc_pos[e];
        const int r = esc_row<R>(pos);
        const int col = cbase + (int)min(esc_tcol<R>(pos), (uint32_t)(a.C - 1));
        const int32_t v = a.esc_val[e];
        if (MODE == 0)
            __builtin_amdgcn_raw_buffer_store_b32(v, ors, (r * a.cols + col) * 4, 0, 0);
        else
            __builtin_amdgcn_raw_buffer_store_b16(to_bf16((float)v * a.step[col]), ors,
                                                  (r * a.cols + col) * 2, 0, 0);
    }
}

// Fixed-rate baseline (rans_gemv.cu:107-131): eight biased nibbles per u32,
// row-major, column 8j+b at bits 4b..4b+3, value = nibble - 8; y = W x' with
// x' = x * step folded by the caller.  A workgroup takes ROWS rows: thread t
// takes the 32-column blocks t, t + blockDim, ..., two blocks per row in
// flight per iteration, loads the 32 x' values of a block once for all its
// rows, and the waves' sums meet in LDS in a fixed order.  Launch shape, from
// a sweep of 1 to 16 rows per workgroup, 1 to 8 waves and one or two blocks
// in flight over the benchmark shapes (rotated copies, us): 8 rows and 4
// waves where both dimensions reach 4096 (25600x5120: 19.9, against 24.0 for
// 16 rows and one block in flight; 5120x17408: 17.8; 5120x5120: 7.2), else
// 4 rows and 8 waves (1536x8960: 5.7), and one wave where a row has at most
// 64 blocks (17920x1536: 6.8, against 13.5 for 16 rows).  Nibbles unpack
// four at a time: masked into the high half of each byte with bit 7
// flipped, a byte holds 16 * (nibble - 8) as a signed 8-bit value, which
// one sign-extending byte conversion reads; the total is scaled by 1/16 at
// the end (exact).
constexpr int kInt4MaxThreads = 512;

// Marks loaded registers as used here: every load above is issued before
// anything after waits for one.  (A memory clobber does not do this for
// const __restrict__ pointers: the compiler may still defer their loads to
// first use, and then waits for each in turn.)
__device__ __forceinline__ void pin(uint4& v) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // one 128-bit operand
    u32x4 t = __builtin_bit_cast(u32x4, v);
    asm volatile("" : "+v"(t));
    v = __builtin_bit_cast(uint4, t);
}
__device__ __forceinline__ void pin(float& v) { asm volatile("" : "+v"(v)); }
template <int N>
__device__ __forceinline__ void pin(float (&v)[4][N]) {
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int k = 0; k < N; k++) pin(v[a][k]);
}

__device__ __forceinline__ float int4_block_dot(uint32_t q, const float (&xs)[8]) {
    // bytes of hi: 16*(n-8) of the odd nibbles (columns 1, 3, 5, 7); of lo:
    // of the even ones (columns 0, 2, 4, 6)
    const uint32_t hi = (q & 0xF0F0F0F0u) ^ 0x80808080u;
    const uint32_t lo = ((q << 4) & 0xF0F0F0F0u) ^ 0x80808080u;
    float a = 0.f;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        a = fmaf((float)(int8_t)(lo >> (8 * k)), xs[2 * k], a);
        a = fmaf((float)(int8_t)(hi >> (8 * k)), xs[2 * k + 1], a);
    }
    return a;
}

// x' of 32-column block j
__device__ __forceinline__ void int4_load_x(const float* __restrict__ x, int j, float (&xs)[4][8]) {
    const float4* xp = reinterpret_cast<const float4*>(x + (int64_t)j * 32);
#pragma unroll
    for (int a = 0; a < 4; a++) {
        const float4 x0 = xp[2 * a], x1 = xp[2 * a + 1];
        xs[a][0] = x0.x; xs[a][1] = x0.y; xs[a][2] = x0.z; xs[a][3] = x0.w;
        xs[a][4] = x1.x; xs[a][5] = x1.y; xs[a][6] = x1.z; xs[a][7] = x1.w;
    }
}

__device__ __forceinline__ float int4_dot(const uint4 q, const float (&xs)[4][8]) {
    return int4_block_dot(q.x, xs[0]) + int4_block_dot(q.y, xs[1]) + int4_block_dot(q.z, xs[2]) +
           int4_block_dot(q.w, xs[3]);
}

template <int ROWS>
__global__ void __launch_bounds__(kInt4MaxThreads) int4_gemv_kernel(const uint32_t* __restrict__ w,
                                                                    const float* __restrict__ x,
                                                                    float* __restrict__ y, int rows,
                                                                    int cols) {
    __shared__ float part[kInt4MaxThreads / 64][ROWS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nthr = blockDim.x;
    const int row0 = blockIdx.x * ROWS;
    const int nblk = cols / 32;
    const int64_t stride = cols / 8;  // u32 per row
    // rows past the end re-read the last row and store nothing
    const uint4* wr[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; r++)
        wr[r] = reinterpret_cast<const uint4*>(w + (int64_t)min(row0 + r, rows - 1) * stride);
    float acc[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; r++) acc[r] = 0.f;
    int j = tid;
    for (; j + nthr < nblk; j += 2 * nthr) {
        uint4 q0[ROWS], q1[ROWS];
#pragma unroll
        for (int r = 0; r < ROWS; r++) {
            q0[r] = wr[r][j];
            q1[r] = wr[r][j + nthr];
        }
        float xs[4][8], xt[4][8];
        int4_load_x(x, j, xs);
        int4_load_x(x, j + nthr, xt);
#pragma unroll
        for (int r = 0; r < ROWS; r++) {
            pin(q0[r]);
            pin(q1[r]);
        }
        pin(xs);
        pin(xt);
#pragma unroll
        for (int r = 0; r < ROWS; r++) acc[r] += int4_dot(q0[r], xs) + int4_dot(q1[r], xt);
    }
    if (j < nblk) {
        // every row's block requested before the first is used: left to
        // itself the compiler issues two and then waits for each of the
        // others in turn (34816x5120: 33.5 against 25.6 us)
        uint4 q[ROWS];
#pragma unroll
        for (int r = 0; r < ROWS; r++) q[r] = wr[r][j];
        float xs[4][8];
        int4_load_x(x, j, xs);
#pragma unroll
        for (int r = 0; r < ROWS; r++) pin(q[r]);
        pin(xs);
#pragma unroll
        for (int r = 0; r < ROWS; r++) acc[r] += int4_dot(q[r], xs);
    }
#pragma unroll
    for (int r = 0; r < ROWS; r++) {
        const float v = wave_sum63(acc[r]);
        if (lane == 63) part[wave][r] = v;
    }
    __syncthreads();
    if (tid < ROWS && row0 + tid < rows) {
        float v = 0.f;
        for (int ww = 0; ww < nthr / 64; ww++) v += part[ww][tid];
        y[row0 + tid] = v * 0.0625f;
    }
}

// Dense bf16 GEMV, the uncompressed comparator: y = W x with W rows x cols
// bf16 row-major, x bf16, y f32 (f32 accumulation), the product F.linear
// computes (bench.py:96 times it through the BLAS library).  A workgroup of
// up to 8 waves takes two rows: thread t takes the 16-byte column chunks t,
// t + blockDim, ..., two chunks per row in flight per iteration, each chunk
// of x (8 values) unpacked once for both rows; the waves' sums meet in LDS
// in a fixed order.  A bf16 value is the high half of its f32, so unpacking
// is a shift or a mask.  Measured over 1 to 8 rows per workgroup, 2 to 16
// waves and 1 to 4 chunks in flight on the benchmark shapes, two rows with
// one wave per 64 chunks (at most 8) and two chunks in flight was the
// fastest or within 5% of it on each (25600x5120: 40 us, 6.5 TB/s; the
// same kernel with 8 rows per workgroup took 51).
constexpr int kBf16MaxThreads = 512;
constexpr int kBf16Rows = 2;

__device__ __forceinline__ float bf16_chunk_dot(const uint4 q, const float (&xs)[8], float a) {
    const uint32_t u[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
        a = fmaf(__uint_as_float(u[k] << 16), xs[2 * k], a);
        a = fmaf(__uint_as_float(u[k] & 0xFFFF0000u), xs[2 * k + 1], a);
    }
    return a;
}

__device__ __forceinline__ void bf16_unpack8(const uint4 v, float (&xs)[8]) {
    const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
        xs[2 * k] = __uint_as_float(u[k] << 16);
        xs[2 * k + 1] = __uint_as_float(u[k] & 0xFFFF0000u);
    }
}

__global__ void __launch_bounds__(kBf16MaxThreads) bf16_gemv_kernel(const uint4* __restrict__ w,
                                                                    const uint4* __restrict__ x,
                                                                    float* __restrict__ y,
                                                                    int rows, int cols) {
    constexpr int ROWS = kBf16Rows;
    __shared__ float part[kBf16MaxThreads / 64][ROWS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nthr = blockDim.x;
    const int row0 = blockIdx.x * ROWS;
    const int nchunk = cols / 8;  // 16-byte chunks per row
    // rows past the end re-read the last row and store nothing
    const uint4* wr[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; r++) wr[r] = w + (int64_t)min(row0 + r, rows - 1) * nchunk;
    float acc[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; r++) acc[r] = 0.f;
    int j = tid;
    for (; j + nthr < nchunk; j += 2 * nthr) {
        uint4 q0[ROWS], q1[ROWS];
        uint4 x0 = x[j], x1 = x[j + nthr];
#pragma unroll
        for (int r = 0; r < ROWS; r++) {
            q0[r] = wr[r][j];
            q1[r] = wr[r][j + nthr];
        }
        // all loads requested before the first use
        pin(x0);
        pin(x1);
#pragma unroll
        for (int r = 0; r < ROWS; r++) {
            pin(q0[r]);
            pin(q1[r]);
        }
        float xs0[8], xs1[8];
        bf16_unpack8(x0, xs0);
        bf16_unpack8(x1, xs1);
#pragma unroll
        for (int r = 0; r < ROWS; r++) acc[r] = bf16_chunk_dot(q1[r], xs1, bf16_chunk_dot(q0[r], xs0, acc[r]));
    }
    if (j < nchunk) {
        uint4 q[ROWS];
#pragma unroll
        for (int r = 0; r < ROWS; r++) q[r] = wr[r][j];
        uint4 xv = x[j];
#pragma unroll
        for (int r = 0; r < ROWS; r++) pin(q[r]);
        pin(xv);
        float xs[8];
        bf16_unpack8(xv, xs);
#pragma unroll
        for (int r = 0; r < ROWS; r++) acc[r] = bf16_chunk_dot(q[r], xs, acc[r]);
    }
#pragma unroll
    for (int r = 0; r < ROWS; r++) {
        const float v = wave_sum63(acc[r]);
        if (lane == 63) part[wave][r] = v;
    }
    __syncthreads();
    if (tid < ROWS && row0 + tid < rows) {
        float v = 0.f;
        for (int ww = 0; ww < nthr / 64; ww++) v += part[ww][tid];
        y[row0 + tid] = v;
    }
}

// ------------------------------------------------------------------ host
WaveLayout wave_layout(const rans_w64_matrix* m) {
    WaveLayout L;
    L.raw_words = (m->max_tile_words + 8 + 7) & ~7;
    L.wave_words = L.raw_words;
    return L;
}

// Dynamic LDS bytes of a launch (the static arrays come on top).
size_t lds_bytes(int waves, const WaveLayout& L) { return (size_t)waves * L.wave_words * 2; }

// Largest byte extent a kernel addresses through one buffer resource
// (an R-row slice of a decoded int32 output): it must fit the 32-bit range.
bool fits_buffer_ranges(const rans_w64_matrix* m) {
    return (int64_t)m->R * m->cols * 4 <= (int64_t)INT32_MAX;
}

bool valid_geometry(const rans_w64_matrix* m) {
    if (!m ||
        (m->flags & ~(RANS_F_WORDS_MASK | RANS_F_NO_ESCAPES | RANS_F_TABLE4 | RANS_F_TABLE8)) ||
        (m->flags & RANS_F_WORDS_MASK) == RANS_F_WORDS_MASK ||
        ((m->flags & RANS_F_TABLE4) && (m->flags & RANS_F_TABLE8)))
        return false;
    if (m->rows <= 0 || m->cols <= 0 || m->R <= 0 || m->C <= 0 || m->S <= 0) return false;
    if (m->rows % m->R || m->cols % m->C || m->C % (64 * m->S)) return false;
    if (m->max_tile_words <= 0 || m->max_tile_words > 65536) return false;
    if (m->max_state_words <= 0 || m->max_state_words > m->max_tile_words) return false;
    return fits_buffer_ranges(m);
}

bool valid_pointers(const rans_w64_matrix* m) {
    return m->words && m->tile_off && m->slen && m->tile_meta && m->table_lds && m->step &&
           m->esc_tileptr && m->esc_pos && m->esc_val;
}

// Waves per GEMV workgroup: the largest divisor of ncb up to kMaxWaves whose
// LDS footprint fits.  Returns 0 when even one wave does not fit.
int gemv_waves(const rans_w64_matrix* m) {
    const int ncb = m->cols / m->C;
    const WaveLayout L = wave_layout(m);
    for (int w = kMaxWaves; w >= 1; w--)
        if (ncb % w == 0 && lds_bytes(w, L) + gemv_static_lds(m->R) <= (size_t)kLdsMax) return w;
    return 0;
}

int device_cus();

// Waves per decode workgroup: among the counts whose LDS fits, the one that
// puts the fewest waves on the busiest CU when the workgroups spread evenly
// over the CUs, the largest such (fewer table copies).
int decode_waves(const rans_w64_matrix* m) {
    const WaveLayout L = wave_layout(m);
    const int64_t ntiles = (int64_t)(m->rows / m->R) * (m->cols / m->C);
    const int cus = device_cus();
    int best = 0;
    int64_t best_load = 0;
    for (int w = 1; w <= kMaxDecodeWaves; w++) {
        if (lds_bytes(w, L) + kDecodeStaticLds > (size_t)kLdsMax) break;
        const int64_t grid = (ntiles + w - 1) / w;
        const int64_t load = cus > 0 ? (grid + cus - 1) / cus * w : -w;
        if (!best || load <= best_load) best = w, best_load = load;
    }
    return best;
}

size_t counters_bytes(const rans_w64_matrix* m) {
    return (((size_t)(m->rows / m->R) * 4 + 255) / 256) * 256;
}

// Opt in to more than 64 KB of LDS once per kernel (bytes dynamic, plus
// static_bytes or more of static __shared__ arrays).
std::mutex g_attr_mu;
const void* g_attr_done[512];
int g_attr_n = 0;

hipError_t ensure_lds(const void* fn, size_t bytes, int static_bytes) {
    if (bytes + static_bytes <= 65536) return hipSuccess;
    std::lock_guard<std::mutex> lk(g_attr_mu);
    for (int i = 0; i < g_attr_n; i++)
        if (g_attr_done[i] == fn) return hipSuccess;
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       kLdsMax - static_bytes);
    if (e == hipSuccess && g_attr_n < 512) g_attr_done[g_attr_n++] = fn;
    return e;
}

// The GEMV kernel for one launch: its address and its static LDS bytes
// (nullptr when no instance is compiled).
struct GemvFn {
    const void* fn;
    int static_lds;
};

template <int R, int S, int B, bool XBF16, bool REFILL, bool GROUP, bool T4, bool ROWS2>
GemvFn gemv_fn_t() {
    return {reinterpret_cast<const void*>(
                &rans_w64_gemv_kernel<R, S, B, XBF16, REFILL, GROUP, T4, ROWS2>),
            gemv_static_lds(R, T4)};
}

// var: bit 0 = bf16 x, bit 1 = refill-only word fetch, bit 2 = grouped
// launch, bit 3 = 4-byte table entries, bit 4 = two tile rows per
// workgroup (bits 2-4 compiled for one state per lane only, at most one of
// them; tiles taller than 16 rows have no paired-row kernels, and of them
// only the 35-row ones have grouped kernels; the batch-8 kernels have only
// the plain and paired-row variants).
template <int R, int S, int B, bool GROUP, bool T4, bool ROWS2>
GemvFn gemv_fn_xf(int var) {
    switch (var & 3) {
        case 0: return gemv_fn_t<R, S, B, false, false, GROUP, T4, ROWS2>();
        case 1: return gemv_fn_t<R, S, B, true, false, GROUP, T4, ROWS2>();
        case 2: return gemv_fn_t<R, S, B, false, true, GROUP, T4, ROWS2>();
        default: return gemv_fn_t<R, S, B, true, true, GROUP, T4, ROWS2>();
    }
}

template <int R, int S, int B>
GemvFn gemv_fn_v(int var) {
    if (var & 28) {
        if constexpr (S == 1) {
            if constexpr ((R <= 16 || R == 35) && B != 8)
                if ((var & 28) == 4) return gemv_fn_xf<R, S, B, true, false, false>(var);
            if constexpr (B != 8)
                if ((var & 28) == 8) return gemv_fn_xf<R, S, B, false, true, false>(var);
            if constexpr (R <= 16)
                if ((var & 28) == 16) return gemv_fn_xf<R, S, B, false, false, true>(var);
        }
        return {nullptr, 0};
    }
    return gemv_fn_xf<R, S, B, false, false, false>(var);
}

template <int R, int S>
GemvFn gemv_fn_b(int B, int var) {
    switch (B) {
        case 1: return gemv_fn_v<R, S, 1>(var);
        case 4: return gemv_fn_v<R, S, 4>(var);
        case 8:
            if constexpr (S == 1 && gemv_max_batch(R) == 8) return gemv_fn_v<R, S, 8>(var);
            return {nullptr, 0};
        default: return {nullptr, 0};
    }
}

template <int R>
GemvFn gemv_fn_s(int S, int B, int var) {
    switch (S) {
        case 1: return gemv_fn_b<R, 1>(B, var);
        case 2: return gemv_fn_b<R, 2>(B, var);
        case 4: return gemv_fn_b<R, 4>(B, var);
        default: return {nullptr, 0};
    }
}

GemvFn gemv_fn(int R, int S, int B, int var) {
    switch (R) {
        case 1: return gemv_fn_s<1>(S, B, var);
        case 2: return gemv_fn_s<2>(S, B, var);
        case 3: return gemv_fn_s<3>(S, B, var);
        case 4: return gemv_fn_s<4>(S, B, var);
        case 8: return gemv_fn_s<8>(S, B, var);
        case 16: return gemv_fn_s<16>(S, B, var);
        case 20: return S == 1 ? gemv_fn_b<20, 1>(B, var) : GemvFn{nullptr, 0};
        case 35: return S == 1 ? gemv_fn_b<35, 1>(B, var) : GemvFn{nullptr, 0};
        default: return {nullptr, 0};
    }
}

int launch_gemv_fn(GemvFn k, const GemvArgs& a, int waves, size_t lds, int grid,
                   hipStream_t stream) {
    if (!k.fn) return RANS_EUNSUPPORTED;
    hipError_t e = ensure_lds(k.fn, lds, k.static_lds);
    if (e != hipSuccess) return (int)e;
    void* args[] = {const_cast<GemvArgs*>(&a)};
    e = hipLaunchKernel(k.fn, dim3(grid), dim3(64 * waves), args, lds, stream);
    const hipError_t last = hipGetLastError();
    return (int)(e != hipSuccess ? e : last);
}

// Workgroups of kernel k that one CU holds at once with `lds` dynamic LDS
// bytes, times the device's CUs (the runtime's occupancy query, which
// counts registers, LDS and wave slots); cached per kernel and shape, since
// launches repeat (the oldest entry is replaced once all 256 are in use).
// 0 when the query fails.
constexpr int kOccEntries = 256;
std::mutex g_occ_mu;
struct OccEntry {
    const void* fn;
    int dev, waves;
    size_t lds;
    int64_t resident;
};
OccEntry g_occ[kOccEntries];
int g_occ_n = 0;     // entries in use
int g_occ_next = 0;  // the next to fill or replace

int64_t resident_workgroups(GemvFn k, int waves, size_t lds) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    std::lock_guard<std::mutex> lk(g_occ_mu);
    for (int i = 0; i < g_occ_n; i++) {
        const OccEntry& o = g_occ[i];
        if (o.fn == k.fn && o.dev == dev && o.waves == waves && o.lds == lds) return o.resident;
    }
    int per_cu = 0, cus = 0;
    if (ensure_lds(k.fn, lds, k.static_lds) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k.fn, 64 * waves, lds) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 0;
    const int64_t resident = (int64_t)per_cu * cus;
    g_occ[g_occ_next] = {k.fn, dev, waves, lds, resident};
    g_occ_next = (g_occ_next + 1) % kOccEntries;
    if (g_occ_n < kOccEntries) g_occ_n++;
    return resident;
}

// CUs of the current device, cached per device; 0 when the query fails.
std::atomic<int> g_cus[64];

int device_cus() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
    if (dev < 64) {
        const int v = g_cus[dev].load(std::memory_order_relaxed);
        if (v > 0) return v;
    }
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 0;
    if (dev < 64) g_cus[dev].store(cus, std::memory_order_relaxed);
    return cus;
}

// Whether a launch takes two tile rows per workgroup.  The 32 KB table copy
// of each workgroup sits on the critical path of a launch the chip holds at
// once (copying it twice made 1536x8960 6% slower); two rows per workgroup
// halve the copies (1536x8960 in 3x2240 tiles: 1.3-2.8% faster over two
// boxes, at 2.25 bits with escapes 5%; in 3x1792 tiles, two rows of five
// waves: 10.05 -> 9.88 us).  Only while the halved grid still gives
// every CU a workgroup (1536x1536 in 8x384 tiles, 192 workgroups, ran 3-5%
// slower as 96), and only where pairing does not raise the most waves a CU
// holds when the workgroups spread evenly: 5120x5120 in 8x1024 tiles (640
// workgroups of 5 waves, 15 waves on the busiest CU) ran 14.5 -> 17.6 us as
// 320 pairs (20).  Single-matrix launches with one state per lane, one
// workgroup per tile row (no split-K), at most 5 waves per row, an even
// number of tile rows and the 8-byte table entries; not tiles taller than
// 16 rows.  The paired workgroup holds both rows' staged blocks, so it is
// only taken when twice the dynamic LDS (lds bytes for one row's waves)
// still fits beside the static arrays.
bool use_rows2(const rans_w64_matrix* m, int n, int v, int waves, int ngroups, int grid,
               size_t lds) {
    if (n != 1 || m->S != 1 || (v & 8) || m->R > 16 || ngroups != 1) return false;
    if (2 * waves > kMaxWavesRows2 || (m->rows / m->R) % 2) return false;
    if (2 * lds + gemv_static_lds(m->R) > (size_t)kLdsMax) return false;
    const int cus = device_cus();
    if (cus <= 0 || grid < 2 * cus) return false;
    const int64_t one = (int64_t)(grid + cus - 1) / cus * waves;
    const int64_t two = (int64_t)(grid / 2 + cus - 1) / cus * 2 * waves;
    return two <= one;
}

// Whether a single-matrix launch of the batch-B kernel runs with the 4-byte
// table entries.  RANS_F_TABLE4 / RANS_F_TABLE8 decide when set.  Otherwise
// only batch 1 with one state per lane does, and only when its grid is more
// than the chip holds at once with the 8-byte entries: there the smaller
// footprint lets more workgroups share a CU (and halves each random table
// read's bytes), while a launch that is resident at once only pays the
// longer decode step (+5% on 1536x8960), and the VALU-bound batch-4 kernel
// the extra instructions (+11% on 25600x5120).
bool use_table4(const rans_w64_matrix* m, int B, int var, int waves, size_t lds, int grid) {
    if (m->flags & RANS_F_TABLE4) return true;
    if ((m->flags & RANS_F_TABLE8) || B != 1 || m->S != 1) return false;
    const int64_t resident = resident_workgroups(gemv_fn(m->R, m->S, B, var), waves, lds);
    return resident > 0 && grid > resident;
}

// Tiles taller than 16 rows take one state per lane.  R = 35 splits rows of
// 8960 = 256 x 35 into 256 tile rows, so that 8960 x 1536 (Qwen2.5-1.5B's
// gate and up projections) runs as 2048 tiles of 35 x 192: two waves on
// every SIMD.  R = 20 is for large matrices, whose launches take more than
// one round of resident workgroups: 25600 rows make 1280 tile rows instead
// of 1600 with R = 16, so the last of the rounds of 768 workgroups is two
// thirds full instead of 8% (25600x5120 at batch 1: 54.8 -> 51.9 us), with
// fewer, longer states (2.923 -> 2.880 bits/weight).
bool supported_rs(int R, int S) {
    return ((R == 1 || R == 2 || R == 3 || R == 4 || R == 8 || R == 16) && (S == 1 || S == 2 || S == 4)) ||
           ((R == 20 || R == 35) && S == 1);
}

template <int R, int S, int MODE>
int launch_decode_t(const DecodeArgs& a, int waves, size_t lds, int grid, hipStream_t stream) {
    const void* fn = reinterpret_cast<const void*>(&rans_w64_decode_kernel<R, S, MODE>);
    hipError_t e = ensure_lds(fn, lds, kDecodeStaticLds);
    if (e != hipSuccess) return (int)e;
    hipLaunchKernelGGL((rans_w64_decode_kernel<R, S, MODE>), dim3(grid), dim3(64 * waves), lds,
                       stream, a);
    return (int)hipGetLastError();
}

template <int MODE>
int dispatch_decode(const DecodeArgs& a, int R, int S, int waves, size_t lds, int grid,
                    hipStream_t st) {
#define VRAMC_DEC_CASE(RR, SS) \
    if (R == RR && S == SS) return launch_decode_t<RR, SS, MODE>(a, waves, lds, grid, st);
#define VRAMC_DEC_R(RR) VRAMC_DEC_CASE(RR, 1) VRAMC_DEC_CASE(RR, 2) VRAMC_DEC_CASE(RR, 4)
    VRAMC_DEC_R(1) VRAMC_DEC_R(2) VRAMC_DEC_R(3) VRAMC_DEC_R(4) VRAMC_DEC_R(8) VRAMC_DEC_R(16)
    VRAMC_DEC_CASE(20, 1) VRAMC_DEC_CASE(35, 1)
#undef VRAMC_DEC_R
#undef VRAMC_DEC_CASE
    return RANS_EUNSUPPORTED;
}

template <int MODE>
int launch_decode_common(const rans_w64_matrix* m, void* out, hipStream_t stream) {
    if (!valid_geometry(m)) return RANS_EGEOMETRY;
    if (!valid_pointers(m) || !out) return RANS_EARG;
    if (!supported_rs(m->R, m->S)) return RANS_EUNSUPPORTED;
    const int waves = decode_waves(m);
    if (!waves) return RANS_EGEOMETRY;
    DecodeArgs a;
    a.words = m->words;
    a.tile_off = m->tile_off;
    a.slen = m->slen;
    a.tile_meta = m->tile_meta;
    a.table_lds = reinterpret_cast<const uint4*>(m->table_lds);
    a.esc_tileptr = m->esc_tileptr;
    a.esc_pos = m->esc_pos;
    a.esc_val = m->esc_val;
    a.step = m->step;
    a.out = out;
    a.rows = m->rows;
    a.cols = m->cols;
    a.C = m->C;
    a.ncb = m->cols / m->C;
    a.ntiles = (m->rows / m->R) * a.ncb;
    a.W = waves;
    a.has_esc = !(m->flags & RANS_F_NO_ESCAPES);
    a.L = wave_layout(m);
    const int grid = (a.ntiles + waves - 1) / waves;
    return dispatch_decode<MODE>(a, m->R, m->S, waves, lds_bytes(waves, a.L), grid, stream);
}

}  // namespace

extern "C" int64_t rans_gemv_workspace_bytes(const rans_w64_matrix* m, int batch) {
    if (!valid_geometry(m) || batch <= 0) return RANS_EGEOMETRY;
    const int waves = gemv_waves(m);
    if (!waves) return RANS_EGEOMETRY;
    const int ngroups = (m->cols / m->C) / waves;
    if (ngroups <= 1) return 0;
    const int bmax = batch >= 2 ? 4 : 1;  // 2 or more run the batch-4 kernel
    return (int64_t)counters_bytes(m) + (int64_t)ngroups * bmax * m->rows * 4;
}

namespace {

// Split-K buffers of one launch: the arrival counters (one per tile row,
// zero between launches) and the partial sums.
struct SplitK {
    uint32_t* counters;
    float* partial;
};

// The split-K buffers in the matrix's own workspace (counters first, then
// the partials), or {nullptr, nullptr} when it is missing or too small.
SplitK workspace_splitk(const rans_w64_matrix* m, int batch) {
    if (!m->workspace || m->workspace_bytes < rans_gemv_workspace_bytes(m, batch))
        return {nullptr, nullptr};
    return {static_cast<uint32_t*>(m->workspace),
            reinterpret_cast<float*>(static_cast<uint8_t*>(m->workspace) + counters_bytes(m))};
}

// One launch of a batch's chunk: nb vectors from vector `first` on the
// batch-B kernel, variant bits v (bit 3: 4-byte table entries, bit 4: two
// tile rows per workgroup).
struct GemvChunk {
    int first, nb, B, v;
};

// The launches a GEMV of `batch` vectors makes, in order, each passed to
// fn (which returns 0 to go on; its first nonzero value is returned).
// Five to eight remaining vectors run as one launch of the batch-8 kernel
// where one is compiled for the tiling and the chunk's variant (one state
// per lane, tiles of at most 8 rows, a single pass over the columns: no
// split-K); otherwise up to 4 run on the batch-4 kernel, and a single
// remaining vector on the batch-1 kernel.  The batch kernels take an
// active-vector count, so a remainder is one launch.  Table entries and
// row pairing are chosen per chunk; t4_image: whether a 4-byte table image
// is (or would be) there to choose.
template <class F>
int plan_gemv(const rans_w64_matrix* m0, int n, int var, int waves, int ngroups, size_t lds,
              int grid, int batch, bool t4_image, F fn) {
    auto variant = [&](int B) {
        int v = var;
        if (n == 1 && t4_image && use_table4(m0, B, var, waves, lds, grid)) v |= 8;
        if (use_rows2(m0, n, v, waves, ngroups, grid, lds)) v |= 16;
        return v;
    };
    int done = 0;
    while (done < batch) {
        const int left = batch - done;
        GemvChunk c{done, 0, 0, 0};
        if (left >= 5 && ngroups == 1) {
            const int v = variant(8);
            if (gemv_fn(m0->R, m0->S, 8, v).fn) c = {done, left >= 8 ? 8 : left, 8, v};
        }
        if (!c.nb) {
            const int B = left >= 2 ? 4 : 1;
            c = {done, left >= 4 ? 4 : (left >= 2 ? left : 1), B, variant(B)};
        }
        const int rc = fn(c);
        if (rc != 0) return rc;
        done += c.nb;
    }
    return 0;
}

// One launch over n matrices that share x (n = 1: any single matrix,
// split-K included, with its buffers in sk; n > 1: a group, validated by
// the caller, never split).
int launch_gemv_common(const rans_w64_matrix* const* ms, int n, const void* x, int x_dtype,
                       int batch, float* const* ys, hipStream_t stream, SplitK sk) {
    const rans_w64_matrix* m0 = ms[0];
    const int waves = gemv_waves(m0);
    if (!waves) return RANS_EGEOMETRY;
    const int ncb0 = m0->cols / m0->C;
    const int ngroups = ncb0 / waves;
    if (ngroups > 1 && (!sk.counters || !sk.partial)) return RANS_EWORKSPACE;
    const bool xbf16 = x_dtype == RANS_X_BF16;
    const size_t xsz = xbf16 ? 2 : 4;
    const int fetch = m0->flags & RANS_F_WORDS_MASK;
    const bool refill = fetch == RANS_F_WORDS_REFILL || (fetch == 0 && m0->R >= 3);
    const int var = (xbf16 ? 1 : 0) | (refill ? 2 : 0) | (n > 1 ? 4 : 0);

    GemvArgs a = {};
    for (int i = 0; i < kMaxGroup; i++) a.wg_begin[i] = INT32_MAX;
    a.cols = m0->cols;
    a.ngroups = ngroups;
    a.W = waves;
    a.counters = ngroups > 1 ? sk.counters : nullptr;
    a.partial = ngroups > 1 ? sk.partial : nullptr;
    int grid = 0;
    a.wave_words = 0;
    for (int i = 0; i < n; i++) {
        const rans_w64_matrix* m = ms[i];
        MatArgs& d = a.mat[i];
        d.words = m->words;
        d.tile_off = m->tile_off;
        d.slen = m->slen;
        d.tile_meta = m->tile_meta;
        d.table_lds = reinterpret_cast<const uint4*>(m->table_lds);
        d.esc_tileptr = m->esc_tileptr;
        d.esc_pos = m->esc_pos;
        d.esc_val = m->esc_val;
        d.step = m->step;
        d.rows = m->rows;
        d.C = m->C;
        d.ncb = m->cols / m->C;
        d.has_esc = !(m->flags & RANS_F_NO_ESCAPES);
        d.raw_words = wave_layout(m).raw_words;
        a.wg_begin[i] = grid;
        grid += (m->rows / m->R) * ngroups;
        if (d.raw_words > a.wave_words) a.wave_words = d.raw_words;
    }
    const size_t lds = (size_t)waves * a.wave_words * 2;

    const bool t4_image = (m0->flags & RANS_F_TABLE4) || m0->table_lds4;
    return plan_gemv(m0, n, var, waves, ngroups, lds, grid, batch, t4_image,
                     [&](const GemvChunk& c) {
        a.x = static_cast<const uint8_t*>(x) + (size_t)c.first * m0->cols * xsz;
        for (int i = 0; i < n; i++) a.mat[i].y = ys[i] + (size_t)c.first * ms[i]->rows;
        a.nb = c.nb;
        if (n == 1)
            a.mat[0].table_lds =
                reinterpret_cast<const uint4*>((c.v & 8) ? m0->table_lds4 : m0->table_lds);
        const bool rows2 = (c.v & 16) != 0;
        a.W = rows2 ? 2 * waves : waves;
        return launch_gemv_fn(gemv_fn(m0->R, m0->S, c.B, c.v), a, a.W, rows2 ? 2 * lds : lds,
                              rows2 ? grid / 2 : grid, stream);
    });
}

bool check_gemv_args(const rans_w64_matrix* m, const void* x, int x_dtype, int batch,
                     const void* y, int& rc) {
    if (!valid_geometry(m)) return rc = RANS_EGEOMETRY, false;
    if (!valid_pointers(m) || !x || !y || batch <= 0) return rc = RANS_EARG, false;
    if (x_dtype != RANS_X_F32 && x_dtype != RANS_X_BF16) return rc = RANS_EARG, false;
    if (!supported_rs(m->R, m->S)) return rc = RANS_EUNSUPPORTED, false;
    if (m->flags & RANS_F_TABLE4) {
        if (!m->table_lds4) return rc = RANS_EARG, false;
        if (m->S != 1) return rc = RANS_EUNSUPPORTED, false;
    }
    return true;
}

}  // namespace

extern "C" int rans_w64_gemv(const rans_w64_matrix* m, const void* x, int x_dtype, int batch,
                                void* y, hipStream_t stream) {
    int rc = 0;
    if (!check_gemv_args(m, x, x_dtype, batch, y, rc)) return rc;
    float* ys[1] = {static_cast<float*>(y)};
    return launch_gemv_common(&m, 1, x, x_dtype, batch, ys, stream, workspace_splitk(m, batch));
}

extern "C" int rans_w64_gemv_group(const rans_w64_matrix* const* ms, int n, const void* x,
                                      int x_dtype, int batch, float* const* ys,
                                      hipStream_t stream) {
    if (!ms || !ys || n <= 0) return RANS_EARG;
    if (n > kMaxGroup) return RANS_EUNSUPPORTED;
    int rc = 0;
    for (int i = 0; i < n; i++)
        if (!check_gemv_args(ms[i], x, x_dtype, batch, ys[i], rc)) return rc;
    const rans_w64_matrix* m0 = ms[0];
    if (m0->S != 1) return RANS_EUNSUPPORTED;
    const int waves = gemv_waves(m0);
    if (!waves) return RANS_EGEOMETRY;
    for (int i = 0; i < n; i++) {
        const rans_w64_matrix* m = ms[i];
        if (m->cols != m0->cols || m->R != m0->R || m->S != m0->S) return RANS_EUNSUPPORTED;
        const int w = gemv_waves(m);
        // one workgroup per tile row (no split-K), the same waves per workgroup
        if (w != waves || (m->cols / m->C) != w) return RANS_EUNSUPPORTED;
        // the group's LDS stride is its largest block region
        if (lds_bytes(waves, wave_layout(m)) + gemv_static_lds(m->R) > (size_t)kLdsMax)
            return RANS_EGEOMETRY;
    }
    return launch_gemv_common(ms, n, x, x_dtype, batch, ys, stream, SplitK{nullptr, nullptr});
}

extern "C" int rans_gemv_table4(const rans_w64_matrix* m, int x_dtype, int batch) {
    if (!valid_geometry(m) || batch <= 0) return RANS_EGEOMETRY;
    if (x_dtype != RANS_X_F32 && x_dtype != RANS_X_BF16) return RANS_EARG;
    if (!supported_rs(m->R, m->S)) return RANS_EUNSUPPORTED;
    if ((m->flags & RANS_F_TABLE4) && m->S != 1) return RANS_EUNSUPPORTED;
    const int waves = gemv_waves(m);
    if (!waves) return RANS_EGEOMETRY;
    const int fetch = m->flags & RANS_F_WORDS_MASK;
    const bool refill = fetch == RANS_F_WORDS_REFILL || (fetch == 0 && m->R >= 3);
    const int var = (x_dtype == RANS_X_BF16 ? 1 : 0) | (refill ? 2 : 0);
    const size_t lds = (size_t)waves * wave_layout(m).raw_words * 2;
    const int ngroups = (m->cols / m->C) / waves;
    const int grid = (m->rows / m->R) * ngroups;
    // the launches rans_w64_gemv makes, were the 4-byte image there
    return plan_gemv(m, 1, var, waves, ngroups, lds, grid, batch, true,
                     [](const GemvChunk& c) { return (c.v & 8) ? 1 : 0; });
}

extern "C" int rans_gemv_rows2(const rans_w64_matrix* m, int x_dtype, int batch) {
    if (!valid_geometry(m) || batch <= 0) return RANS_EGEOMETRY;
    if (x_dtype != RANS_X_F32 && x_dtype != RANS_X_BF16) return RANS_EARG;
    if (!supported_rs(m->R, m->S)) return RANS_EUNSUPPORTED;
    const int waves = gemv_waves(m);
    if (!waves) return RANS_EGEOMETRY;
    const int fetch = m->flags & RANS_F_WORDS_MASK;
    const bool refill = fetch == RANS_F_WORDS_REFILL || (fetch == 0 && m->R >= 3);
    const int var = (x_dtype == RANS_X_BF16 ? 1 : 0) | (refill ? 2 : 0);
    const size_t lds = (size_t)waves * wave_layout(m).raw_words * 2;
    const int ngroups = (m->cols / m->C) / waves;
    const int grid = (m->rows / m->R) * ngroups;
    // the launches rans_w64_gemv makes (table entries first: paired rows
    // need the 8-byte ones, then the pairing)
    const bool t4_image = (m->flags & RANS_F_TABLE4) || m->table_lds4;
    return plan_gemv(m, 1, var, waves, ngroups, lds, grid, batch, t4_image,
                     [](const GemvChunk& c) { return (c.v & 16) ? 1 : 0; });
}

extern "C" int rans_w64_decode(const rans_w64_matrix* m, void* out_bf16, hipStream_t stream) {
    return launch_decode_common<1>(m, out_bf16, stream);
}

extern "C" int rans_w64_decode_codes(const rans_w64_matrix* m, int32_t* out, hipStream_t stream) {
    return launch_decode_common<0>(m, out, stream);
}

extern "C" int launch_int4_gemv(const void* w, const void* x, void* y, int rows, int cols,
                                hipStream_t stream) {
    if (!w || !x || !y || rows <= 0 || cols <= 0) return RANS_EARG;
    // 16-byte loads of w rows and x blocks
    if (cols % 32 || ((uintptr_t)w | (uintptr_t)x) % 16) return RANS_EGEOMETRY;
    // rows per workgroup and waves as measured (see the kernel)
    const int nblk = cols / 32;
    const bool large = rows >= 4096 && cols >= 4096;
    const int waves = nblk <= 64 ? 1 : large ? 4 : 8;
    const auto* wp = static_cast<const uint32_t*>(w);
    const auto* xp = static_cast<const float*>(x);
    auto* yp = static_cast<float*>(y);
    const dim3 block(64 * waves);
    if (large)
        hipLaunchKernelGGL(int4_gemv_kernel<8>, dim3((rows + 7) / 8), block, 0, stream, wp, xp, yp, rows, cols);
    else
        hipLaunchKernelGGL(int4_gemv_kernel<4>, dim3((rows + 3) / 4), block, 0, stream, wp, xp, yp, rows, cols);
    return (int)hipGetLastError();
}

extern "C" int bf16_gemv(const void* w, const void* x, void* y, int rows, int cols,
                         hipStream_t stream) {
    if (!w || !x || !y || rows <= 0 || cols <= 0) return RANS_EARG;
    if (cols % 8 || ((uintptr_t)w | (uintptr_t)x) % 16) return RANS_EGEOMETRY;
    // one wave per 64 chunks of a row, at most 8; two rows per workgroup
    const int nchunk = cols / 8;
    const int waves = std::min(kBf16MaxThreads / 64, (nchunk + 63) / 64);
    const dim3 grid((rows + kBf16Rows - 1) / kBf16Rows), block(64 * waves);
    hipLaunchKernelGGL(bf16_gemv_kernel, grid, block, 0, stream, static_cast<const uint4*>(w),
                       static_cast<const uint4*>(x), static_cast<float*>(y), rows, cols);
    return (int)hipGetLastError();
}

// ------------------------------------------------ allocation-free GEMV entry
// rans_w64_gemv_noalloc runs split-K launches with the partial sums and the
// arrival counters in this file-scope array instead of the matrix's
// workspace: one array per GPU, held until the process ends, shared by every
// call on that GPU (so calls that overlap on one GPU race).  Layout: the
// counters (RANS_SCRATCH_COUNTER_BYTES, one u32 per tile row, zero between
// launches), then the partials.  Host code never passes the array's name to
// a kernel: on the host it is a stand-in, not a device address.  Its device
// address comes from hipGetSymbolAddress, once per device.
namespace {

static __device__ __align__(256) uint8_t scratch[RANS_SCRATCH_BYTES];

__global__ void __launch_bounds__(256) zero_u32_kernel(uint32_t* p, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = 0u;
}

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
uint8_t* g_scratch_ptr[kScratchDevices];

// The scratch array's device address on the current device.  The first call
// on a device looks it up and clears the counters with a fill kernel on
// `stream` (a kernel, so that a call under graph capture records a kernel
// node); every GEMV leaves the counters it used at zero again.
int scratch_base(hipStream_t stream, uint8_t** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= kScratchDevices) return RANS_EUNSUPPORTED;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int)e;
        if (!p) return RANS_EARG;
        constexpr int n = RANS_SCRATCH_COUNTER_BYTES / 4;
        hipLaunchKernelGGL(zero_u32_kernel, dim3((n + 255) / 256), dim3(256), 0, stream,
                           static_cast<uint32_t*>(p), n);
        e = hipGetLastError();
        if (e != hipSuccess) return (int)e;
        g_scratch_ptr[dev] = static_cast<uint8_t*>(p);
    }
    *out = g_scratch_ptr[dev];
    return 0;
}

}  // namespace

extern "C" int rans_w64_gemv_noalloc(const rans_w64_matrix* m, const void* x, int x_dtype,
                                     int batch, void* y, hipStream_t stream) {
    int rc = 0;
    if (!check_gemv_args(m, x, x_dtype, batch, y, rc)) return rc;
    const int64_t need = rans_gemv_workspace_bytes(m, batch);
    if (need < 0) return (int)need;
    SplitK sk{nullptr, nullptr};
    if (need > 0) {
        // the sizes are checked before anything touches the device
        const int64_t counters = (int64_t)(m->rows / m->R) * 4;
        const int64_t partials = need - (int64_t)counters_bytes(m);
        if (counters > RANS_SCRATCH_COUNTER_BYTES ||
            partials > (int64_t)RANS_SCRATCH_BYTES - RANS_SCRATCH_COUNTER_BYTES)
            return RANS_ESCRATCH;
        uint8_t* base = nullptr;
        rc = scratch_base(stream, &base);
        if (rc != 0) return rc;
        sk = {reinterpret_cast<uint32_t*>(base),
              reinterpret_cast<float*>(base + RANS_SCRATCH_COUNTER_BYTES)};
    }
    float* ys[1] = {static_cast<float*>(y)};
    return launch_gemv_common(&m, 1, x, x_dtype, batch, ys, stream, sk);
}
