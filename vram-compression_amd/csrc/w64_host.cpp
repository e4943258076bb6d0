// Host side of the w64 stream format: static table build, the wavefront-
// interleaved multi-state encoder, and a host decoder.  Plain C++17, no GPU
// calls; built into librans_hip.so next to the kernels.
//
// The coder arithmetic is the reference's (kernel/rans.py:13-16, 62-98,
// 101-123); the layout is this library's (see include/vramc_rans.h).
#include <algorithm>
#include <array>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/vramc_rans.h"

namespace {

constexpr uint32_t kScaleBits = 12;
constexpr uint32_t kM = 1u << kScaleBits;
constexpr uint32_t kRansL = 1u << 16;
constexpr int kEsc = 0;

struct Encoded {
    std::vector<uint16_t> words;
    std::vector<uint32_t> tile_off;
    std::vector<uint32_t> tile_meta;  // per tile: length base | blob words << 16
    std::vector<uint8_t> slen;        // per state: length - base | state exponent << 4
    uint32_t table[kM];
    int64_t freq[256];
    int64_t counts[256] = {0};  // symbol counts over the matrix
    std::vector<int32_t> esc_tileptr;
    std::vector<uint16_t> esc_pos;  // tile-local index c*R + r
    std::vector<int16_t> esc_val;
    int64_t payload_words = 0;
    int32_t max_tile_words = 0;
    int32_t max_state_words = 0;  // longest state stream, counting the tile padding
};

// Initial decoder state x (in [2^16, 2^32)) as its exponent e = floor(log2 x)
// - 16 (0..15) and the 16 + e bits below its leading one.
int state_exponent(uint32_t x) { return 31 - __builtin_clz(x) - 16; }

// Appends the low n bits of v (n <= 31) to a little-endian bit stream of
// 16-bit words at bit offset pos.
void put_bits(std::vector<uint16_t>& w, size_t first, uint64_t pos, uint32_t v, int n) {
    for (int i = 0; i < n; i++, pos++) {
        const size_t k = first + (size_t)(pos >> 4);
        if ((v >> i) & 1u) w[k] |= (uint16_t)(1u << (pos & 15));
    }
}

// Runs fn(i) for i in [0, n) on up to nthreads threads, static blocks.
template <typename F>
void parallel_for(int64_t n, int nthreads, F fn) {
    if (nthreads <= 1 || n < 2) {
        for (int64_t i = 0; i < n; i++) fn(i);
        return;
    }
    nthreads = (int)std::min<int64_t>(nthreads, n);
    std::vector<std::thread> pool;
    for (int t = 0; t < nthreads; t++) {
        pool.emplace_back([=, &fn] {
            const int64_t lo = n * t / nthreads, hi = n * (t + 1) / nthreads;
            for (int64_t i = lo; i < hi; i++) fn(i);
        });
    }
    for (auto& th : pool) th.join();
}

}  // namespace

namespace {

// The table from symbol counts (n = their sum).
int table_from_counts(const int64_t* counts, int64_t n, int64_t* freq, int64_t* cum,
                      uint32_t* table) {
    if (n <= 0) return RANS_ECODES;
    // Same quantisation as rans.py:36-44: round-half-even of count*M/total in
    // double precision, floor of 1 for present symbols, then move the rounding
    // residue onto the first largest bin.
    int64_t sum = 0;
    for (int s = 0; s < 256; s++) {
        int64_t f = 0;
        if (counts[s]) {
            const double v = std::nearbyint(((double)counts[s] * (double)kM) / (double)n);
            f = v < 1.0 ? 1 : (int64_t)v;
        }
        freq[s] = f;
        sum += f;
    }
    while (sum != (int64_t)kM) {
        const int64_t diff = (int64_t)kM - sum;
        int big = 0;
        for (int s = 1; s < 256; s++)
            if (freq[s] > freq[big]) big = s;
        const int64_t adj = diff < 0 ? std::max<int64_t>(diff, 1 - freq[big]) : diff;
        freq[big] += adj;
        sum += adj;
    }
    for (int s = 0; s < 256; s++)
        if (freq[s] >= (int64_t)kM) return RANS_ECODES;
    int64_t c = 0;
    for (int s = 0; s < 256; s++) {
        if (cum) cum[s] = c;
        for (int64_t k = 0; k < freq[s]; k++)
            table[c + k] = (uint32_t)s | ((uint32_t)freq[s] << 8) | ((uint32_t)k << 20);
        c += freq[s];
    }
    return 0;
}

}  // namespace

extern "C" int rans_build_table(const uint8_t* sym, int64_t n, int64_t* freq, int64_t* cum,
                                uint32_t* table) {
    if (n <= 0 || !sym) return RANS_ECODES;
    int64_t counts[256] = {0};
    for (int64_t i = 0; i < n; i++) counts[sym[i]]++;
    return table_from_counts(counts, n, freq, cum, table);
}

extern "C" int rans_table_lds(const uint32_t* table, uint32_t* out) {
    if (!table || !out) return RANS_EARG;
    for (uint32_t i = 0; i < kM; i++) {
        const uint32_t e = table[i];
        const uint32_t sym = e & 0xFFu;
        const uint32_t code = sym == 0 ? 0u : (uint32_t)((int32_t)sym - 128);
        out[2 * i] = ((e >> 8) & 0xFFFu) | (code << 24);
        out[2 * i + 1] = e >> 20;
    }
    return 0;
}

extern "C" int rans_table_lds4(const uint32_t* table, uint32_t* out) {
    if (!table || !out) return RANS_EARG;
    for (uint32_t i = 0; i < kM; i++) {
        const uint32_t e = table[i];
        const uint32_t sym = e & 0xFFu;
        const uint32_t code = sym == 0 ? 0u : (uint32_t)((int32_t)sym - 128);
        out[i] = ((e >> 8) & 0xFFFu) | ((e >> 20) << 12) | (code << 24);
    }
    return 0;
}

extern "C" int rans_w64_encode(const int32_t* codes, int32_t rows, int32_t cols, int32_t R,
                               int32_t C, int32_t S, int32_t nthreads, void** handle,
                               int64_t* info) {
    if (!codes || !handle || !info || rows <= 0 || cols <= 0 || R <= 0 || C <= 0 || S <= 0)
        return RANS_EARG;
    if (rows % R || cols % C || C % (64 * S)) return RANS_EGEOMETRY;
    if ((int64_t)R * C > 65536) return RANS_EGEOMETRY;  // 16-bit tile-local escape positions
    const int64_t N = (int64_t)rows * cols;
    auto* E = new Encoded();

    // Symbols and their counts, in parallel over row blocks (per-block
    // histograms summed in block order); the escape side table is collected
    // per tile below.
    std::vector<uint8_t> sym((size_t)N);
    const int nth = nthreads > 0 ? nthreads : 1;
    const int64_t nblk = std::min<int64_t>((int64_t)nth * 4, rows);
    std::vector<std::array<int64_t, 256>> hist((size_t)nblk);
    std::vector<int> wide((size_t)nblk, 0);  // a code beyond the 16-bit escape values
    parallel_for(nblk, nth, [&](int64_t b) {
        std::array<int64_t, 256>& h = hist[(size_t)b];
        h.fill(0);
        const int64_t lo = (int64_t)rows * b / nblk * cols, hi = (int64_t)rows * (b + 1) / nblk * cols;
        for (int64_t i = lo; i < hi; i++) {
            const int32_t v = codes[i];
            const uint8_t y = v >= -127 && v <= 127 ? (uint8_t)(v + 128) : (uint8_t)kEsc;
            wide[(size_t)b] |= v < -32768 || v > 32767;
            sym[(size_t)i] = y;
            h[y]++;
        }
    });
    for (int w : wide)
        if (w) {
            delete E;
            return RANS_ECODES;
        }
    for (const auto& h : hist)
        for (int y = 0; y < 256; y++) E->counts[y] += h[(size_t)y];

    int64_t cum[256];
    if (table_from_counts(E->counts, N, E->freq, cum, E->table) != 0) {
        delete E;
        return RANS_ECODES;
    }

    const int32_t ncb = cols / C, nrb = rows / R;
    const int64_t ntiles = (int64_t)nrb * ncb;
    const int32_t nst = 64 * S;
    const int32_t nk = C / nst;
    const int64_t n = (int64_t)nk * R;  // symbols per state

    std::vector<std::vector<uint16_t>> blocks((size_t)ntiles);
    E->tile_meta.assign((size_t)ntiles, 0);
    E->slen.assign((size_t)(ntiles * nst), 0);
    std::vector<int64_t> payload((size_t)ntiles, 0);
    std::vector<int> too_big((size_t)ntiles, 0);
    std::vector<int32_t> longest((size_t)ntiles, 0);
    std::vector<std::vector<uint16_t>> tesc_pos((size_t)ntiles);
    std::vector<std::vector<int16_t>> tesc_val((size_t)ntiles);

    const int64_t* freq = E->freq;
    parallel_for(ntiles, nthreads > 0 ? nthreads : 1, [&](int64_t t) {
        const int32_t rb = (int32_t)(t / ncb), cb = (int32_t)(t % ncb);
        std::vector<uint8_t> seq((size_t)n);
        std::vector<uint16_t> emitted((size_t)n);
        // each state's words in decode order and its initial decoder state
        std::vector<std::vector<uint16_t>> dec((size_t)nst);
        std::vector<uint32_t> x0((size_t)nst);
        for (int32_t j = 0; j < nst; j++) {
            const int32_t s = j / 64, l = j % 64;
            int64_t i = 0;
            for (int32_t k = 0; k < nk; k++) {
                const int64_t col = (int64_t)cb * C + 64 * ((int64_t)S * k + s) + l;
                for (int32_t r = 0; r < R; r++)
                    seq[(size_t)i++] = sym[(size_t)(((int64_t)rb * R + r) * cols + col)];
            }
            // Reverse encode (rans.py:76-83): renormalise when x >= 2^20*f,
            // then x = (x/f)<<12 + x%f + cum.  x stays below 2^32.
            uint32_t x = kRansL;
            int64_t cnt = 0;
            for (int64_t q = n - 1; q >= 0; q--) {
                const uint32_t f = (uint32_t)freq[seq[(size_t)q]];
                const uint32_t c = (uint32_t)cum[seq[(size_t)q]];
                if (x >= (f << 20)) {
                    emitted[(size_t)cnt++] = (uint16_t)(x & 0xFFFF);
                    x >>= 16;
                }
                x = ((x / f) << kScaleBits) + (x % f) + c;
            }
            x0[(size_t)j] = x;
            std::vector<uint16_t>& d = dec[(size_t)j];
            d.resize((size_t)cnt);
            for (int64_t q = 0; q < cnt; q++) d[(size_t)q] = emitted[(size_t)(cnt - 1 - q)];
            payload[(size_t)t] += cnt;
        }
        // Lengths against the tile's base: each stored length is base + a
        // 4-bit delta, so where the lengths spread over more than 16 values
        // the streams below max - 15 are padded with zero words (never read)
        // up to it.
        int32_t lo = INT32_MAX, hi = 0;
        for (const auto& d : dec) {
            lo = std::min(lo, (int32_t)d.size());
            hi = std::max(hi, (int32_t)d.size());
        }
        const int32_t base = std::max(lo, hi - 15);
        if (base > 255) too_big[(size_t)t] = 1;
        // Block: the initial states' mantissas bit-packed (state j's 16 + e_j
        // bits after those of states 0..j-1, little endian), then the
        // streams in state order, then at least one pad word (the decoder
        // reads one word ahead), rounded up to 8 words (16-byte loads).
        uint64_t nbits = 0;
        for (int32_t j = 0; j < nst; j++) nbits += 16 + state_exponent(x0[(size_t)j]);
        const size_t blob_words = (size_t)((nbits + 15) / 16);
        std::vector<uint16_t>& blk = blocks[(size_t)t];
        blk.assign(blob_words, 0);
        uint64_t pos = 0;
        for (int32_t j = 0; j < nst; j++) {
            const int e = state_exponent(x0[(size_t)j]);
            put_bits(blk, 0, pos, x0[(size_t)j] - (1u << (16 + e)), 16 + e);
            pos += 16 + e;
        }
        int32_t lmax = 0;
        for (int32_t j = 0; j < nst; j++) {
            const std::vector<uint16_t>& d = dec[(size_t)j];
            const int32_t len = std::max((int32_t)d.size(), base);
            blk.insert(blk.end(), d.begin(), d.end());
            blk.resize(blk.size() + (size_t)(len - (int32_t)d.size()), 0);
            E->slen[(size_t)(t * nst + j)] =
                (uint8_t)((len - base) | state_exponent(x0[(size_t)j]) << 4);
            lmax = std::max(lmax, len);
        }
        const size_t streams_end = blk.size();
        const size_t padded = (blk.size() + 1 + 7) & ~(size_t)7;
        if (padded > 65535) too_big[(size_t)t] = 1;
        blk.resize(padded, 0);
        // the last stream as staged: up to the end of the padded block
        const int32_t last = std::max((int32_t)dec[(size_t)nst - 1].size(), base);
        longest[(size_t)t] = std::max(lmax, (int32_t)(padded - streams_end) + last);
        E->tile_meta[(size_t)t] = (uint32_t)(base & 0xFF) | (uint32_t)blob_words << 16;
        // the tile's escapes in column order, rows ascending within a column
        for (int32_t c = 0; c < C; c++)
            for (int32_t r = 0; r < R; r++) {
                const int64_t i = ((int64_t)rb * R + r) * cols + (int64_t)cb * C + c;
                if (sym[(size_t)i] == kEsc) {
                    tesc_pos[(size_t)t].push_back((uint16_t)(c * R + r));
                    tesc_val[(size_t)t].push_back((int16_t)codes[i]);
                }
            }
    });
    for (int64_t t = 0; t < ntiles; t++) {
        if (too_big[(size_t)t]) {
            delete E;
            return RANS_ETILE;
        }
    }

    E->tile_off.assign((size_t)ntiles + 1, 0);
    int64_t total = 0;
    for (int64_t t = 0; t < ntiles; t++) {
        E->tile_off[(size_t)t] = (uint32_t)total;
        total += (int64_t)blocks[(size_t)t].size();
        E->max_tile_words = std::max<int32_t>(E->max_tile_words, (int32_t)blocks[(size_t)t].size());
        E->max_state_words = std::max<int32_t>(E->max_state_words, longest[(size_t)t]);
        E->payload_words += payload[(size_t)t];
    }
    if (total > 0xFFFFFFFFll) {
        delete E;
        return RANS_ETILE;
    }
    E->tile_off[(size_t)ntiles] = (uint32_t)total;
    E->esc_tileptr.assign((size_t)ntiles + 1, 0);
    int64_t nesc = 0;
    for (int64_t t = 0; t < ntiles; t++) {
        E->esc_tileptr[(size_t)t] = (int32_t)nesc;
        nesc += (int64_t)tesc_pos[(size_t)t].size();
    }
    if (nesc > 0x7FFFFFFFll) {
        delete E;
        return RANS_ETILE;
    }
    E->esc_tileptr[(size_t)ntiles] = (int32_t)nesc;
    E->esc_pos.reserve((size_t)nesc);
    E->esc_val.reserve((size_t)nesc);
    for (int64_t t = 0; t < ntiles; t++) {
        E->esc_pos.insert(E->esc_pos.end(), tesc_pos[(size_t)t].begin(), tesc_pos[(size_t)t].end());
        E->esc_val.insert(E->esc_val.end(), tesc_val[(size_t)t].begin(), tesc_val[(size_t)t].end());
    }
    E->words.resize((size_t)total);
    parallel_for(ntiles, nthreads > 0 ? nthreads : 1, [&](int64_t t) {
        std::memcpy(E->words.data() + E->tile_off[(size_t)t], blocks[(size_t)t].data(),
                    blocks[(size_t)t].size() * sizeof(uint16_t));
    });

    info[0] = total;
    info[1] = ntiles;
    info[2] = ntiles * nst;
    info[3] = (int64_t)E->esc_pos.size();
    info[4] = E->max_tile_words;
    info[5] = E->payload_words;
    info[6] = E->max_state_words;
    *handle = E;
    return 0;
}

extern "C" int rans_w64_encode_fetch(void* handle, uint16_t* words, uint32_t* tile_off,
                                     uint32_t* tile_meta, uint8_t* slen, uint32_t* table,
                                     int64_t* freq, int32_t* esc_tileptr, uint16_t* esc_pos,
                                     int16_t* esc_val) {
    if (!handle) return RANS_EARG;
    auto* E = static_cast<Encoded*>(handle);
    auto put = [](auto* dst, const auto& v) {
        if (dst && !v.empty()) std::memcpy(dst, v.data(), v.size() * sizeof(v[0]));
    };
    put(words, E->words);
    put(tile_off, E->tile_off);
    put(tile_meta, E->tile_meta);
    put(slen, E->slen);
    put(esc_tileptr, E->esc_tileptr);
    put(esc_pos, E->esc_pos);
    put(esc_val, E->esc_val);
    if (table) std::memcpy(table, E->table, sizeof(E->table));
    if (freq) std::memcpy(freq, E->freq, sizeof(E->freq));
    return 0;
}

extern "C" int rans_w64_encode_counts(void* handle, int64_t* counts) {
    if (!handle || !counts) return RANS_EARG;
    std::memcpy(counts, static_cast<Encoded*>(handle)->counts, sizeof(int64_t) * 256);
    return 0;
}

extern "C" void rans_w64_encode_free(void* handle) { delete static_cast<Encoded*>(handle); }

extern "C" int rans_w64_decode_host(const rans_w64_matrix* m, int32_t* out) {
    if (!m || !out || !m->words || !m->tile_off || !m->slen || !m->tile_meta || !m->table)
        return RANS_EARG;
    const int32_t rows = m->rows, cols = m->cols, R = m->R, C = m->C, S = m->S;
    if (R <= 0 || C <= 0 || S <= 0 || rows % R || cols % C || C % (64 * S)) return RANS_EGEOMETRY;
    const int32_t ncb = cols / C, nrb = rows / R, nst = 64 * S, nk = C / nst;
    const int64_t ntiles = (int64_t)nrb * ncb;
    const int64_t nwords = m->tile_off[ntiles];
    // Tiles decode independently, on up to 16 threads; each stops at its
    // first failure, and the failure of the lowest tile is returned (what a
    // tile-by-tile decode would return).
    auto decode_tile = [&](int64_t t) -> int {
        const int32_t rb = (int32_t)(t / ncb), cb = (int32_t)(t % ncb);
        const int64_t blk = m->tile_off[t], blk_end = m->tile_off[t + 1];
        const int32_t base = (int32_t)(m->tile_meta[t] & 0xFF);
        const int64_t blob_words = m->tile_meta[t] >> 16;
        if (blk_end < blk || blk + blob_words > blk_end || blk_end > nwords) return RANS_EARG;
        // the initial states' mantissas, then the streams in state order
        uint64_t bit = 0;
        int64_t start = blk + blob_words;
        for (int32_t j = 0; j < nst; j++) {
            const int32_t s = j / 64, l = j % 64;
            const int64_t sid = t * nst + j;
            const int32_t e = m->slen[sid] >> 4, nb = 16 + e;
            if (bit + (uint64_t)nb > (uint64_t)blob_words * 16) return RANS_EARG;
            uint32_t mant = 0;
            for (int i = 0; i < nb; i++, bit++)
                mant |= (uint32_t)((m->words[blk + (int64_t)(bit >> 4)] >> (bit & 15)) & 1u) << i;
            uint32_t st = (1u << nb) | mant;
            const int64_t len = base + (m->slen[sid] & 15);
            int64_t p = start;
            for (int32_t k = 0; k < nk; k++) {
                const int64_t col = (int64_t)cb * C + 64 * ((int64_t)S * k + s) + l;
                for (int32_t r = 0; r < R; r++) {
                    const uint32_t e = m->table[st & (kM - 1)];
                    st = ((e >> 8) & 0xFFFu) * (st >> kScaleBits) + (e >> 20);
                    if (st < kRansL) {
                        if (p >= start + len) return RANS_EARG;
                        st = (st << 16) | m->words[p++];
                    }
                    out[((int64_t)rb * R + r) * cols + col] = (int32_t)(e & 0xFF) - 128;
                }
            }
            if (st != kRansL) return (int)(sid + 1 > 0x7fffffff ? 0x7fffffff : sid + 1);
            // the state consumed exactly its stored length, or stopped short of
            // a stream padded up to its tile's base
            if (p - start != len && len != base) return RANS_EARG;
            start += len;
        }
        return start < blk_end ? 0 : RANS_EARG;  // at least one pad word follows
    };
    std::vector<int> err((size_t)ntiles, 0);
    const int nth = (int)std::min<unsigned>(16, std::max(1u, std::thread::hardware_concurrency()));
    parallel_for(ntiles, nth, [&](int64_t t) { err[(size_t)t] = decode_tile(t); });
    for (int64_t t = 0; t < ntiles; t++)
        if (err[(size_t)t]) return err[(size_t)t];
    // The escape symbol decodes to kEsc-128; the side table must name exactly
    // those positions: the same count, each entry inside its tile on an
    // escape symbol, strictly ascending within the tile (so none twice).
    int64_t nesc_stream = 0;
    for (int64_t i = 0; i < (int64_t)rows * cols; i++) nesc_stream += out[i] == kEsc - 128;
    const int64_t nesc = m->esc_tileptr ? m->esc_tileptr[ntiles] : 0;
    if (nesc != nesc_stream) return RANS_EARG;
    if (!nesc) return 0;
    if (!m->esc_pos || !m->esc_val || m->esc_tileptr[0] != 0) return RANS_EARG;
    for (int64_t t = 0; t < ntiles; t++) {
        const int32_t rb = (int32_t)(t / ncb), cb = (int32_t)(t % ncb);
        const int32_t lo = m->esc_tileptr[t], hi = m->esc_tileptr[t + 1];
        if (lo > hi || hi > nesc) return RANS_EARG;
        for (int32_t e = lo; e < hi; e++) {
            const int32_t pos = m->esc_pos[e];
            const int32_t r = pos % R, c = pos / R;
            if (c >= C || (e > lo && pos <= m->esc_pos[e - 1])) return RANS_EARG;
            int32_t* o = out + ((int64_t)rb * R + r) * cols + (int64_t)cb * C + c;
            if (*o != kEsc - 128) return RANS_EARG;
            *o = m->esc_val[e];
        }
    }
    return 0;
}

// The reference's own 32-lane layout (kernel/rans.py:55-98), for the
// reference-format entry points (launch_rans_gemv / launch_rans_decode): one
// stream per lane of 32-column tiles, lanes in tile order, each stream its
// final encoder state as two words and then its renormalisation words in
// decode order, 8 zero words after the last stream.  The table is built with
// the same quantisation as the w64 encoder, from symbols code + 128 (codes in
// [-128, 127], no escapes).  Lanes are encoded on up to nthreads threads; the
// output does not depend on the thread count.
extern "C" int rans_ref32_encode(const int32_t* codes, int32_t rows, int32_t cols, int32_t R,
                                 int32_t C, int32_t nthreads, uint16_t* words, int64_t words_cap,
                                 uint32_t* offs, uint32_t* table, int64_t* info) {
    if (!codes || !words || !offs || !table || !info || rows <= 0 || cols <= 0 || R <= 0 ||
        C <= 0)
        return RANS_EARG;
    if (rows % R || cols % C || C % 32) return RANS_EGEOMETRY;
    const int64_t N = (int64_t)rows * cols;
    const int32_t ncb = cols / C;
    const int64_t lanes = (int64_t)(rows / R) * ncb * 32;
    const int64_t n = (int64_t)(C / 32) * R;  // symbols per lane
    if (words_cap < 2 * lanes + N + 8) return RANS_EARG;  // the longest possible output
    int64_t counts[256] = {0};
    for (int64_t i = 0; i < N; i++) {
        const int32_t v = codes[i];
        if (v < -128 || v > 127) return RANS_ECODES;
        counts[v + 128]++;
    }
    int64_t freq[256], cum[256];
    if (table_from_counts(counts, N, freq, cum, table) != 0) return RANS_ECODES;

    // each lane's emitted words (in encode order) and final state
    std::vector<std::vector<uint16_t>> emitted((size_t)lanes);
    std::vector<uint32_t> final_state((size_t)lanes);
    const int nth = nthreads > 0 ? nthreads : 1;
    parallel_for(lanes, nth, [&](int64_t li) {
        const int64_t t = li / 32, l = li % 32;
        const int64_t rb = t / ncb, cb = t % ncb;
        std::vector<uint16_t>& out = emitted[(size_t)li];
        out.reserve((size_t)(n / 2 + 4));
        uint64_t x = kRansL;
        for (int64_t i = n - 1; i >= 0; i--) {
            const int64_t k = i / R, r = i % R;  // symbol i = k*R + r
            const int32_t s = codes[(rb * R + r) * cols + cb * C + 32 * k + l] + 128;
            const uint64_t f = (uint64_t)freq[s], c = (uint64_t)cum[s];
            if (x >= ((uint64_t)1 << 20) * f) {
                out.push_back((uint16_t)(x & 0xFFFFu));
                x >>= 16;
            }
            x = ((x / f) << kScaleBits) + x % f + c;
        }
        final_state[(size_t)li] = (uint32_t)x;
    });
    int64_t pos = 0, payload = 0;
    for (int64_t li = 0; li < lanes; li++) {
        const std::vector<uint16_t>& out = emitted[(size_t)li];
        offs[li] = (uint32_t)pos;
        words[pos++] = (uint16_t)(final_state[(size_t)li] >> 16);
        words[pos++] = (uint16_t)(final_state[(size_t)li] & 0xFFFFu);
        for (size_t j = out.size(); j-- > 0;) words[pos++] = out[j];
        payload += (int64_t)out.size();
    }
    for (int j = 0; j < 8; j++) words[pos++] = 0;
    info[0] = pos;
    info[1] = payload;
    return 0;
}
