// The reference's own stream format decoded on MI355X (gfx950), behind the
// reference's two rANS entry points with their argument lists and meaning
// (launch_rans_gemv / launch_rans_decode, rans_gemv.cu:146-162):
//   - words, offs and table as the reference's encode returns them
//     (kernel/rans.py:62-98): lane j of tile (rb, cb) has one stream starting
//     at words[offs[32*(rb*ncb + cb) + j]], its 32-bit initial state in the
//     first two words, then its renormalisation words; it holds columns
//     cb*C + j + 32k for k < C/32, all R rows of the tile, symbol order
//     k-major, r-minor (rans_gemv.cu:7-11);
//   - table[slot] = sym | freq<<8 | (slot-cum)<<20, code = sym - 128
//     (rans_gemv.cu:32-37);
//   - the GEMV takes the host-folded f32 x' = x*step and writes y when one
//     column tile spans the matrix, else adds into y, which the caller has
//     zeroed (rans.py:141-146);
//   - the decode writes bf16(code * step[c]) row-major.
// A binding written for the reference therefore runs unchanged on this
// library.  The format has few, long streams (one per 32 columns of a tile,
// 2240 symbols each at the reference's 1536x8960 tiling), so it is a
// compatibility path: the w64 layout that rans_w64_gemv runs decodes the same
// matrix far faster.
//
// Shape on gfx950: one wavefront decodes 64 consecutive reference lanes (two
// 32-lane tiles).  The reference's encoder lays the streams out in lane
// order, so a wave's streams are one span of words, which the wave copies
// into its LDS slot before decoding; each renormalisation then reads LDS.  A
// span longer than the slot is decoded from global memory instead (slower,
// same results).  The span ends at the next wave's first offset, or, for the
// last wave, after the longest stream its last lane can have (two state
// words plus one word per symbol), cut at the end of the allocation that
// holds `words` (queried on the host): no copy reads outside it.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>

#include "../../include/vramc_rans.h"

namespace {

constexpr uint32_t kRefM = 4096;
constexpr uint32_t kRefL = 1u << 16;
constexpr int kRefMaxWaves = 4;
constexpr int kRefLdsMax = 160 * 1024;
constexpr int kRefStaticLds = 8 * (int)kRefM;  // the 8-byte table image
constexpr int kRefSlotMax = 64 * 1024;         // LDS words per wave at most
constexpr int kRefBufWord3 = 0x00020000;       // buffer resource word 3 for raw loads

struct Ref32Args {
    const uint16_t* words;
    const uint32_t* offs;
    const uint32_t* table;
    const float* xs;      // GEMV: x' = x*step; decode: step
    void* out;            // GEMV: y, f32 [rows]; decode: bf16 [rows][cols]
    int64_t words_avail;  // 16-bit words from `words` to the end of its allocation
    int rows, cols, C, ncb;
    int nlanes;   // (rows/R) * (cols/C) * 32
    int slot;     // LDS words per wave (a multiple of 8)
    int words16;  // `words` is 16-byte aligned: stage with direct global->LDS copies
};

__device__ __forceinline__ uint32_t ref_lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
__device__ __forceinline__ uint32_t ref_lds_u16(uint32_t a) {
    return *(const __attribute__((address_space(3))) uint16_t*)(uintptr_t)a;
}

// v from lane (dpp CTRL) in the rows of ROWS, 0 in the others
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ float ref_dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWS, 0xF, false));
}

// Sum over each 32-lane half of the wave (one reference tile each), in a
// fixed order: the totals land in lanes 31 and 63.
__device__ __forceinline__ float ref_half_sum(float v) {
    v += ref_dpp<0xB1>(v);        // quad_perm [1,0,3,2]
    v += ref_dpp<0x4E>(v);        // quad_perm [2,3,0,1]
    v += ref_dpp<0x141>(v);       // row_half_mirror: sums of 8
    v += ref_dpp<0x140>(v);       // row_mirror: 16-lane row sums
    v += ref_dpp<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
    return v;
}

__device__ __forceinline__ uint16_t ref_bf16(float f) {
    return __builtin_bit_cast(uint16_t, (__bf16)f);
}

// One decode step (rans_gemv.cu:32-37) on the 8-byte image {freq | code<<24,
// slot-cum}, software-pipelined: e holds the table entry of this symbol,
// read in the previous step, and the next entry is read as soon as the new
// state exists, ahead of the word refill; the next word w is read ahead.
// Words in LDS: the select form (the read-ahead word is long back when the
// select needs it).
__device__ __forceinline__ int32_t ref_step_lds(uint32_t& st, uint32_t& ad, uint32_t& w, uint2& e,
                                                const uint2* tab) {
    const uint2 cur = e;
    const uint32_t ns = __umul24(cur.x, st >> 12) + cur.y;
    const bool need = ns < kRefL;
    st = need ? ((ns << 16) | w) : ns;
    e = tab[st & (kRefM - 1)];
    if (need) {
        ad += 2u;
        w = ref_lds_u16(ad);
    }
    return (int32_t)cur.x >> 24;
}

// The same step with the words in global memory.  The renormalised state is
// formed inside the branch (an asm statement the compiler cannot hoist), so
// a wave waits for a lane's read-ahead word only when that lane consumes it.
__device__ __forceinline__ int32_t ref_step_global(uint32_t& st, uint32_t& p, uint32_t& w, uint2& e,
                                                   const uint2* tab, __amdgpu_buffer_rsrc_t wrs) {
    const uint2 cur = e;
    const uint32_t ns = __umul24(cur.x, st >> 12) + cur.y;
    st = ns;
    if (ns < kRefL) {
        asm volatile("v_lshl_or_b32 %0, %1, 16, %2" : "=v"(st) : "v"(ns), "v"(w));
        p += 1u;
        w = __builtin_amdgcn_raw_buffer_load_b16(wrs, (int)(p * 2u), 0, 0);
    }
    e = tab[st & (kRefM - 1)];
    return (int32_t)cur.x >> 24;
}

template <int R, bool DECODE>
__global__ void __launch_bounds__(64 * kRefMaxWaves) ref32_kernel(Ref32Args a) {
    __shared__ __align__(16) uint2 tab[kRefM];
    extern __shared__ __align__(16) uint16_t ref_dyn[];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int W = blockDim.x >> 6;
    // the reference's packed table as the 8-byte image; code = sym - 128 for
    // every symbol of this format (it has no escapes)
    for (int i = threadIdx.x; i < (int)kRefM; i += blockDim.x) {
        const uint32_t e = a.table[i];
        tab[i] = make_uint2(((e >> 8) & 0xFFFu) | (((e & 0xFFu) - 128u) << 24), e >> 20);
    }
    const int g = blockIdx.x * W + wave;  // this wave's group of 64 lanes
    const int base = g * 64;
    const bool live = base < a.nlanes;  // wave-uniform
    const int L = base + lane;
    const bool active = live && L < a.nlanes;
    uint16_t* slot = ref_dyn + (size_t)wave * a.slot;
    const int nsym = (a.C / 32) * R;

    // The span of the wave's streams, words [w0, w1): from its first lane's
    // offset (rounded down to a 16-byte chunk) to the next wave's first
    // offset, or past the last lane's longest possible stream; never past
    // the end of the allocation.
    int64_t w0 = 0, w1 = 0;
    if (live) {
        w0 = ((int64_t)a.offs[base] >> 3) << 3;
        const int64_t end = base + 64 < a.nlanes
                                ? (int64_t)a.offs[base + 64] + 1
                                : (int64_t)a.offs[a.nlanes - 1] + 3 + nsym;
        w1 = min(end, a.words_avail);
    }
    // staged when the span (plus the read-ahead slack) fits the slot and
    // every lane's stream starts inside it (offsets in lane order, as the
    // reference's encoder writes them; otherwise the global path)
    const uint32_t p0 = active ? a.offs[L] : 0u;
    const bool inside = !active || ((int64_t)p0 >= w0 && (int64_t)p0 < w1);
    const bool staged = live && w1 > w0 && (w1 - w0) + 8 <= a.slot &&
                        __builtin_amdgcn_ballot_w64(!inside) == 0;
    if (staged) {
        // whole 16-byte chunks that end inside the allocation, then the last
        // few words one by one: every load lies in range
        const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint16_t*>(a.words) + w0, 0,
            (int)min((a.words_avail - w0) * 2, (int64_t)0x7FFFFFFF), kRefBufWord3);
        const int nfull = (int)min((w1 - w0 + 7) >> 3, (a.words_avail - w0) >> 3);
        if (a.words16) {
            // 16-byte aligned words: direct global->LDS copies, all issued
            // before the one wait (lane i's 16 bytes land at base + 16*i)
            const uint4* src = reinterpret_cast<const uint4*>(a.words + w0);
            for (int j0 = 0; j0 < nfull; j0 += 64)
                if (j0 + lane < nfull)
                    __builtin_amdgcn_global_load_lds(
                        src + j0 + lane,
                        (__attribute__((address_space(3))) void*)(slot + 8 * j0), 16, 0, 0);
        } else {
            // through registers, four chunks in flight per lane
            using V4 = decltype(__builtin_amdgcn_raw_buffer_load_b128(srs, 0, 0, 0));
            for (int j = lane; j < nfull; j += 256) {
                V4 v[4];
#pragma unroll
                for (int u = 0; u < 4; u++)
                    if (j + 64 * u < nfull)
                        v[u] = __builtin_amdgcn_raw_buffer_load_b128(srs, (j + 64 * u) * 16, 0, 0);
#pragma unroll
                for (int u = 0; u < 4; u++)
                    if (j + 64 * u < nfull)
                        *reinterpret_cast<V4*>(slot + 8 * (j + 64 * u)) = v[u];
            }
        }
        const int ntail = (int)(w1 - w0) - 8 * nfull;  // < 8
        if (lane < ntail)
            slot[8 * nfull + lane] =
                __builtin_amdgcn_raw_buffer_load_b16(srs, (8 * nfull + lane) * 2, 0, 0);
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the direct copies have landed
    __syncthreads();

    // this lane's tile: rows rb*R.., columns cb*C + l + 32k
    const int t = L >> 5, l = L & 31;
    const int rb = t / a.ncb, cb = t - (t / a.ncb) * a.ncb;
    const int col0 = cb * a.C + l;
    const int nk = a.C / 32;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.f;
    if (active) {
        uint16_t* outb = static_cast<uint16_t*>(a.out);
        auto emit = [&](int k, int r, int32_t code, float xv) {
            if constexpr (DECODE)
                outb[(int64_t)(rb * R + r) * a.cols + col0 + 32 * k] = ref_bf16((float)code * xv);
            else
                acc[r] = fmaf((float)code, xv, acc[r]);
            // consumed here: otherwise the compiler sinks the conversions
            // and FMAs past the refill branches and reorders the reads
            asm volatile("" : "+v"(acc[r]));
        };
        if (staged) {
            uint32_t ad = ref_lds_addr(slot + (p0 - (uint32_t)w0));
            uint32_t st = (ref_lds_u16(ad) << 16) | ref_lds_u16(ad + 2u);
            ad += 4u;
            uint32_t w = ref_lds_u16(ad);
            uint2 e = tab[st & (kRefM - 1)];
            float xn = a.xs[col0];
            for (int k = 0; k < nk; k++) {
                const float xv = xn;
                xn = a.xs[col0 + 32 * min(k + 1, nk - 1)];
#pragma unroll
                for (int r = 0; r < R; r++) emit(k, r, ref_step_lds(st, ad, w, e, tab), xv);
            }
        } else {
            // ranged from the wave's first offset, so the byte offsets stay
            // small; a lane whose offset lies below it (offsets out of lane
            // order) reads out of range, i.e. zeros, never another buffer
            const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<uint16_t*>(a.words) + w0, 0,
                (int)min(max(a.words_avail - w0, (int64_t)0) * 2, (int64_t)0x7FFFFFFF),
                kRefBufWord3);
            uint32_t p = p0 - (uint32_t)w0;
            uint32_t st = ((uint32_t)__builtin_amdgcn_raw_buffer_load_b16(wrs, (int)(p * 2u), 0, 0)
                           << 16) |
                          __builtin_amdgcn_raw_buffer_load_b16(wrs, (int)(p * 2u + 2u), 0, 0);
            p += 2u;
            uint32_t w = __builtin_amdgcn_raw_buffer_load_b16(wrs, (int)(p * 2u), 0, 0);
            uint2 e = tab[st & (kRefM - 1)];
            for (int k = 0; k < nk; k++) {
                const float xv = a.xs[col0 + 32 * k];
#pragma unroll
                for (int r = 0; r < R; r++) emit(k, r, ref_step_global(st, p, w, e, tab, wrs), xv);
            }
        }
    }
    if constexpr (!DECODE) {
        float* y = static_cast<float*>(a.out);
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float v = ref_half_sum(acc[r]);
            if ((lane & 31) == 31 && active) {
                if (a.ncb == 1)
                    y[rb * R + r] = v;
                else
                    atomicAdd(&y[rb * R + r], v);
            }
        }
    }
}

// Opt in to the dynamic LDS once per kernel.
std::mutex g_ref_attr_mu;
const void* g_ref_attr_done[16];
int g_ref_attr_n = 0;

hipError_t ref_ensure_lds(const void* fn, size_t bytes) {
    if (bytes + kRefStaticLds <= 65536) return hipSuccess;
    std::lock_guard<std::mutex> lk(g_ref_attr_mu);
    for (int i = 0; i < g_ref_attr_n; i++)
        if (g_ref_attr_done[i] == fn) return hipSuccess;
    const hipError_t e =
        hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, kRefLdsMax - kRefStaticLds);
    if (e == hipSuccess && g_ref_attr_n < 16) g_ref_attr_done[g_ref_attr_n++] = fn;
    return e;
}

template <int R, bool DECODE>
int ref32_launch(const Ref32Args& a, int W, hipStream_t stream) {
    const void* fn = reinterpret_cast<const void*>(&ref32_kernel<R, DECODE>);
    const size_t dyn = (size_t)W * a.slot * 2;
    if (const hipError_t e = ref_ensure_lds(fn, dyn); e != hipSuccess) return (int)e;
    const int nwaves = (a.nlanes + 63) / 64;
    hipLaunchKernelGGL((ref32_kernel<R, DECODE>), dim3((nwaves + W - 1) / W), dim3(64 * W), dyn,
                       stream, a);
    return (int)hipGetLastError();
}

// Checks, then the launch; R outside the reference's set returns -1 as the
// reference does (rans_gemv.cu:137-144), before anything else is touched.
template <bool DECODE>
int ref32_entry(int R, const void* words, const void* offs, const void* table, const void* xs,
                void* out, int rows, int cols, int C, hipStream_t stream) {
    if (R != 1 && R != 2 && R != 4 && R != 8 && R != 16) return RANS_EUNSUPPORTED;
    if (!words || !offs || !table || !xs || !out) return RANS_EARG;
    if (rows <= 0 || cols <= 0 || C <= 0 || C % 32 || rows % R || cols % C) return RANS_EGEOMETRY;
    const int64_t nlanes = (int64_t)(rows / R) * (cols / C) * 32;
    if (nlanes > INT32_MAX - 64 || (int64_t)rows * cols > ((int64_t)1 << 40)) return RANS_EGEOMETRY;
    hipDeviceptr_t base = nullptr;
    size_t size = 0;
    if (const hipError_t e =
            hipMemGetAddressRange(&base, &size, const_cast<hipDeviceptr_t>(words));
        e != hipSuccess)
        return (int)e;
    const int64_t avail =
        ((int64_t)(static_cast<const uint8_t*>(base) + size - static_cast<const uint8_t*>(words))) / 2;
    if (avail <= 0) return RANS_EARG;

    Ref32Args a;
    a.words = static_cast<const uint16_t*>(words);
    a.offs = static_cast<const uint32_t*>(offs);
    a.table = static_cast<const uint32_t*>(table);
    a.xs = static_cast<const float*>(xs);
    a.out = out;
    a.words_avail = avail;
    a.words16 = ((uintptr_t)words & 15) == 0;
    a.rows = rows;
    a.cols = cols;
    a.C = C;
    a.ncb = cols / C;
    a.nlanes = (int)nlanes;
    // LDS slot per wave: 64 streams at up to 5 bits per symbol, plus the last
    // wave's bound on its last stream, within what the CU holds; spans above
    // the slot take the global-memory path
    const int64_t nsym = (int64_t)(C / 32) * R;
    int64_t slot = 64 * (nsym * 5 / 16 + 4) + nsym + 24;
    slot = (slot + 7) / 8 * 8;
    if (slot > kRefSlotMax) slot = kRefSlotMax;
    a.slot = (int)slot;
    int W = (kRefLdsMax - kRefStaticLds) / (int)(slot * 2);
    W = W < 1 ? 1 : (W > kRefMaxWaves ? kRefMaxWaves : W);
    switch (R) {
        case 1: return ref32_launch<1, DECODE>(a, W, stream);
        case 2: return ref32_launch<2, DECODE>(a, W, stream);
        case 4: return ref32_launch<4, DECODE>(a, W, stream);
        case 8: return ref32_launch<8, DECODE>(a, W, stream);
        default: return ref32_launch<16, DECODE>(a, W, stream);
    }
}

}  // namespace

extern "C" int launch_rans_gemv(int R, const void* words, const void* offs, const void* table,
                                const void* x, void* y, int rows, int cols, int C,
                                hipStream_t stream) {
    return ref32_entry<false>(R, words, offs, table, x, y, rows, cols, C, stream);
}

extern "C" int launch_rans_decode(int R, const void* words, const void* offs, const void* table,
                                  const void* step, void* out_bf16, int rows, int cols, int C,
                                  hipStream_t stream) {
    return ref32_entry<true>(R, words, offs, table, step, out_bf16, rows, cols, C, stream);
}
