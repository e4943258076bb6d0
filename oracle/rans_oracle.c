/*
 * ORACLE -- test infrastructure only.  This file is the CPU checker for the
 * entropy-coded GEMV; nothing in the shipped library links, loads or calls it.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it.
 *
 * Plain-C restatement of the reference coder (kernel/rans.py of
 * snuri00/vram-compression), written from its documented arithmetic:
 *   - 32-bit decoder state in [2^16, 2^32), 16-bit renormalisation words,
 *     12-bit probabilities (M = 4096), symbol = code + 128      rans.py:13-16
 *   - table build with round-half-even + first-argmax fix-up      rans.py:34-51
 *   - per-lane reverse encoder, stream = [x>>16, x&0xFFFF] + reversed
 *     emitted words, 8 pad words at the end                       rans.py:62-98
 *   - per-lane decoder with final-state check                     rans.py:101-121
 *   - dense dequant GEMV y = codes @ (x * step), in float64       rans_gemv.cu:4-6
 *
 * Lanes here are generic "independent streams": the caller supplies the
 * symbol matrix already in lane order (lanes x n, lane-major), so the same
 * routines check both the reference 32-lane layout and any other layout that
 * uses the same per-stream arithmetic.
 *
 * Every function returns 0 on success and a negative value on a violated
 * precondition, so Python callers turn failures into exceptions.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORC_SCALE_BITS 12
#define ORC_M (1u << ORC_SCALE_BITS)
#define ORC_RANS_L (1u << 16)

/* rans.py:34-51.  counts over 256 symbols; freq = max(1, round_half_even(
 * count*M/total)) for present symbols; while sum != M adjust the first
 * argmax bin (a negative diff is clamped so the bin stays >= 1); reject a
 * distribution whose largest bin reaches M.  table[slot] packs
 * sym | freq<<8 | (slot-cum)<<20.  Returns -1 for an empty input, -2 for a
 * degenerate (single-symbol) distribution. */
int orc_build_table(const uint8_t* sym, int64_t n, int64_t* freq, int64_t* cum,
                    uint32_t* table) {
    if (n <= 0) return -1;
    int64_t counts[256];
    memset(counts, 0, sizeof counts);
    for (int64_t i = 0; i < n; i++) counts[sym[i]]++;
    const double total = (double)n;
    int64_t sum = 0;
    for (int s = 0; s < 256; s++) {
        freq[s] = 0;
        if (counts[s] > 0) {
            /* numpy: counts[present] * M / counts.sum(), float64, then np.round */
            double v = nearbyint(((double)counts[s] * (double)ORC_M) / total);
            freq[s] = v < 1.0 ? 1 : (int64_t)v;
        }
        sum += freq[s];
    }
    while (sum != (int64_t)ORC_M) {
        int64_t diff = (int64_t)ORC_M - sum;
        int imax = 0;
        for (int s = 1; s < 256; s++)
            if (freq[s] > freq[imax]) imax = s; /* first maximum, as np.argmax */
        int64_t adj;
        if (diff < 0) {
            int64_t floor_adj = 1 - freq[imax];
            adj = diff > floor_adj ? diff : floor_adj;
        } else {
            adj = diff;
        }
        freq[imax] += adj;
        sum += adj;
    }
    for (int s = 0; s < 256; s++)
        if (freq[s] >= (int64_t)ORC_M) return -2;
    int64_t c = 0;
    for (int s = 0; s < 256; s++) {
        cum[s] = c;
        for (int64_t k = 0; k < freq[s]; k++)
            table[c + k] = (uint32_t)s | ((uint32_t)freq[s] << 8) | ((uint32_t)k << 20);
        c += freq[s];
    }
    return 0;
}

/* rans.py:76-83 for one lane: encode syms[0..n) in reverse.  Emitted words are
 * written to out[] in emission order; returns the count, and the final state
 * through *xfinal.  Arithmetic in 64 bits as the reference does (uint64). */
static int64_t encode_one(const uint8_t* syms, int64_t n, const int64_t* freq,
                          const int64_t* cum, uint16_t* out, uint64_t* xfinal) {
    uint64_t x = ORC_RANS_L;
    int64_t cnt = 0;
    for (int64_t i = n - 1; i >= 0; i--) {
        const uint64_t f = (uint64_t)freq[syms[i]];
        const uint64_t c = (uint64_t)cum[syms[i]];
        if (x >= ((uint64_t)1 << 20) * f) {
            out[cnt++] = (uint16_t)(x & 0xFFFF);
            x >>= 16;
        }
        x = ((x / f) << ORC_SCALE_BITS) + (x % f) + c;
    }
    *xfinal = x;
    return cnt;
}

/* Word count per lane without materialising the stream (rans.py:76-83, the
 * `cnt` array).  lanes x n lane-major symbols.  counts[l] = emitted words. */
int orc_count_words(const uint8_t* S, int64_t lanes, int64_t n, const int64_t* freq,
                    const int64_t* cum, int64_t* counts) {
    if (lanes < 0 || n < 0) return -1;
    for (int64_t l = 0; l < lanes; l++) {
        const uint8_t* syms = S + l * n;
        if (n > 0 && freq[syms[0]] == 0) return -3;
        uint64_t x = ORC_RANS_L;
        int64_t cnt = 0;
        for (int64_t i = n - 1; i >= 0; i--) {
            const uint64_t f = (uint64_t)freq[syms[i]];
            if (f == 0) return -3;
            const uint64_t c = (uint64_t)cum[syms[i]];
            if (x >= ((uint64_t)1 << 20) * f) {
                cnt++;
                x >>= 16;
            }
            x = ((x / f) << ORC_SCALE_BITS) + (x % f) + c;
        }
        counts[l] = cnt;
    }
    return 0;
}

/* rans.py:62-98: the reference stream layout.  words must hold
 * sum(counts)+2*lanes+8 entries (orc_count_words gives the counts); offs gets
 * one u32 word offset per lane.  Returns -3 for a symbol with zero frequency. */
int orc_encode_lanes(const uint8_t* S, int64_t lanes, int64_t n, const int64_t* freq,
                     const int64_t* cum, uint16_t* words, int64_t words_cap,
                     uint32_t* offs) {
    if (lanes < 0 || n < 0) return -1;
    uint16_t* tmp = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)(n > 0 ? n : 1));
    if (!tmp) return -4;
    int64_t pos = 0;
    for (int64_t l = 0; l < lanes; l++) {
        const uint8_t* syms = S + l * n;
        for (int64_t i = 0; i < n; i++)
            if (freq[syms[i]] == 0) { free(tmp); return -3; }
        uint64_t x;
        const int64_t cnt = encode_one(syms, n, freq, cum, tmp, &x);
        if (pos + cnt + 2 + 8 > words_cap) { free(tmp); return -5; }
        offs[l] = (uint32_t)pos;
        words[pos] = (uint16_t)(x >> 16);
        words[pos + 1] = (uint16_t)(x & 0xFFFF);
        for (int64_t k = 0; k < cnt; k++) words[pos + 2 + k] = tmp[cnt - 1 - k];
        pos += cnt + 2;
    }
    for (int k = 0; k < 8; k++) words[pos + k] = 0; /* rans.py:87 pad */
    free(tmp);
    return 0;
}

/* rans.py:101-121 for streams whose initial state is given separately:
 * decode n symbols from each lane.  state0[l] is the initial 32-bit state,
 * start[l] the word index of the lane's first renormalisation word.  Writes
 * raw symbols (0..255) lane-major into out.  Returns -(l+1) for the first
 * lane whose final state is not 2^16 or that would read past nwords. */
int orc_decode_streams(const uint16_t* words, int64_t nwords, const uint32_t* state0,
                       const int64_t* start, int64_t lanes, int64_t n,
                       const uint32_t* table, uint8_t* out) {
    for (int64_t l = 0; l < lanes; l++) {
        uint64_t st = state0[l];
        int64_t p = start[l];
        uint8_t* o = out + l * n;
        for (int64_t i = 0; i < n; i++) {
            const uint32_t e = table[st & (ORC_M - 1)];
            st = (uint64_t)((e >> 8) & 0xFFF) * (st >> ORC_SCALE_BITS) + (e >> 20);
            if (st < ORC_RANS_L) {
                if (p < 0 || p >= nwords) return (int)-(l + 1);
                st = (st << 16) | words[p];
                p++;
            }
            o[i] = (uint8_t)(e & 0xFF);
        }
        if (st != ORC_RANS_L) return (int)-(l + 1);
    }
    return 0;
}

/* rans.py:101-121 on the reference layout: each lane's stream begins with the
 * two state words at offs[l]. */
int orc_decode_lanes(const uint16_t* words, int64_t nwords, const uint32_t* offs,
                     int64_t lanes, int64_t n, const uint32_t* table, uint8_t* out) {
    uint32_t* st0 = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)(lanes > 0 ? lanes : 1));
    int64_t* start = (int64_t*)malloc(sizeof(int64_t) * (size_t)(lanes > 0 ? lanes : 1));
    if (!st0 || !start) { free(st0); free(start); return -4; }
    for (int64_t l = 0; l < lanes; l++) {
        const int64_t p = offs[l];
        if (p + 1 >= nwords) { free(st0); free(start); return (int)-(l + 1); }
        st0[l] = ((uint32_t)words[p] << 16) | words[p + 1];
        start[l] = p + 2;
    }
    const int rc = orc_decode_streams(words, nwords, st0, start, lanes, n, table, out);
    free(st0);
    free(start);
    return rc;
}

/* rans_gemv.cu:4-6 semantics in float64: y[b,r] = sum_c codes[r,c]*x[b,c]*step[c]. */
int orc_gemv_f64(const int32_t* codes, int64_t rows, int64_t cols, const double* x,
                 int64_t batch, const double* step, double* y) {
    double* xs = (double*)malloc(sizeof(double) * (size_t)(cols > 0 ? cols : 1));
    if (!xs) return -4;
    for (int64_t b = 0; b < batch; b++) {
        for (int64_t c = 0; c < cols; c++) xs[c] = x[b * cols + c] * step[c];
        for (int64_t r = 0; r < rows; r++) {
            const int32_t* row = codes + r * cols;
            double acc = 0.0;
            for (int64_t c = 0; c < cols; c++) acc += (double)row[c] * xs[c];
            y[b * rows + r] = acc;
        }
    }
    free(xs);
    return 0;
}
