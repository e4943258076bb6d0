/*
 * vramc_rans.h -- C ABI of librans_hip.so: entropy-coded (rANS) weight
 * matrices decoded inside a batch-1 GEMV on MI355X (gfx950).
 *
 * Drop-in boundary for kernel/rans.py + kernel/rans_gemv.cu of
 * snuri00/vram-compression.  The reference's C ABI (rans_gemv.cu:146-170)
 * passes a flat list of raw pointers for its 32-lane stream; the wavefront
 * stream format here carries more buffers (per-tile offsets, per-state
 * initial states, an escape side table, the per-column step), so they travel
 * in one plain-C descriptor, rans_w64_matrix, passed by pointer.  Every
 * pointer in it is a device pointer owned by the caller (the Python wrapper
 * keeps the tensors alive, as rans.py:134-137 does); the library keeps no
 * state between calls except the per-process kernel attribute setup.
 *
 * Conventions kept from the reference:
 *   - launches are asynchronous on the caller's stream (hipStream_t, e.g.
 *     torch.cuda.current_stream().cuda_stream);
 *   - the return value is 0 on success, a hipError_t value for a launch
 *     error (hipGetLastError after the launch), or a negative value for a
 *     rejected argument (the reference returns -1 for an unsupported R,
 *     rans_gemv.cu:143).  No call synchronises.
 *
 * Stream format "w64" (all integers little endian):
 *   - W (rows x cols) holds integer codes; W_real[r,c] = code[r,c]*step[c].
 *   - The matrix is cut into tiles of R rows x C columns, tile t = rb*(cols/C)+cb.
 *     A tile is decoded by one 64-lane wavefront with S rANS states per lane;
 *     state j = s*64 + l decodes, for k < C/(64*S) and r < R (k-major,
 *     r-minor), the code at row rb*R+r, column cb*C + 64*(S*k+s) + l.
 *   - Coder arithmetic is the reference's (rans.py:13-16, rans_gemv.cu:32-37):
 *     32-bit state, 16-bit renormalisation words, 12-bit probabilities,
 *     table[slot] = sym | freq<<8 | (slot-cum)<<20, sym = code + 128.
 *   - Symbol 0 is the escape: codes outside [-127, 127] are coded as symbol 0
 *     and their values live in a side table kept per tile: tile t's entries
 *     are esc_pos/esc_val[esc_tileptr[t] .. esc_tileptr[t+1]), esc_pos =
 *     c*R + r (16 bits) for the code at tile row r, tile column c (row
 *     rb*R+r, column cb*C+c), strictly ascending within the tile, so a
 *     tile's entries run in column order; esc_val is the code (16 bits).
 *     Hence R*C <= 65536 and escape codes within [-32768, 32767].
 *   - words: all tile blocks concatenated; tile t's block is
 *     words[tile_off[t] .. tile_off[t+1]), a multiple of 8 words with at least
 *     one trailing pad word.  It opens with the tile's initial decoder states
 *     (blob_words words), then holds the streams of its 64*S states in state
 *     order (each state's renormalisation words in decode order).
 *   - tile_meta[t] = base | blob_words << 16 and, per state j, slen[t*64*S+j]
 *     = (len_j - base) | e_j << 4: state j's stream is len_j words and starts
 *     blob_words + len_0 + .. + len_{j-1} words into the block.  Where a
 *     tile's lengths spread over more than 16 values, the shorter streams are
 *     padded with zero words (never read) up to base.
 *   - State j's initial value x_j in [2^16, 2^32) is stored as its exponent
 *     e_j = floor(log2 x_j) - 16 (in slen) and its 16 + e_j bits below the
 *     leading one, at bit b_j = (16 + e_0) + .. + (16 + e_{j-1}) of the
 *     block read as a little-endian bit stream (bit i is bit i%16 of word
 *     i/16).  32 bits of state and 8 of length became 8 + 16 + e_j bits.
 *   - A stream of n symbols has at most 0.75n+1 words (12 bits per symbol at
 *     most); the bases fit a byte for states of up to 338 symbols
 *     (R*C/(64*S)).
 */
#ifndef VRAMC_RANS_H
#define VRAMC_RANS_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* x dtype codes for rans_w64_gemv */
#define RANS_X_F32 0
#define RANS_X_BF16 1

/* rejected-argument return values */
#define RANS_EUNSUPPORTED (-1) /* R, S or batch without a compiled kernel: the GPU entry
                                  points take R in {1, 2, 3, 4, 8, 16} with S in {1, 2, 4},
                                  and R in {20, 35} with S = 1 (the encoder and host
                                  decoder take any R <= 256) */
#define RANS_EGEOMETRY (-2)    /* shape not divisible, or tile too large for LDS */
#define RANS_EWORKSPACE (-3)   /* split-K workspace missing or too small */
#define RANS_EARG (-4)         /* null pointer or negative size */
#define RANS_ECODES (-5)       /* encoder: degenerate or empty symbol distribution, or a
                                  code outside [-32768, 32767] */
#define RANS_ETILE (-6)        /* encoder: a tile block exceeds 65535 words, or a tile's
                                  length base 255 */
#define RANS_ESCRATCH (-7)     /* rans_w64_gemv_noalloc: the launch needs more split-K
                                  scratch than the library holds (RANS_SCRATCH_BYTES) */

/* The scratch array of rans_w64_gemv_noalloc, one per GPU: arrival counters
 * (one u32 per tile row, so at most 16384 tile rows), then split-K partial
 * sums (4 bytes per output row, column group and batch row of a batch-4
 * chunk, so at most 4128768 bytes of them). */
#define RANS_SCRATCH_BYTES (4 << 20)
#define RANS_SCRATCH_COUNTER_BYTES (64 << 10)

/* rans_w64_matrix.flags.  Word fetch (bits 0-1): how the GEMV fetches
 * renormalisation words; the decoded values are identical, only speed
 * differs; 0 = library default (REFILL for R >= 3, ALWAYS otherwise). */
#define RANS_F_WORDS_ALWAYS 1 /* every lane re-reads its next word each step */
#define RANS_F_WORDS_REFILL 2 /* only lanes that consumed their word fetch the next */
#define RANS_F_WORDS_MASK 3
#define RANS_F_NO_ESCAPES 4   /* the side table is empty: kernels skip it (a promise; a
                                 matrix with escapes decodes them as 0 under this flag) */
/* Table entries of the GEMV (bits 3-4; same results, different speed).  With
 * neither flag the library picks: the 4-byte entries (table_lds4, when set)
 * for a batch-1 launch with S = 1 whose workgroups do not all fit on the chip
 * at once with the 8-byte ones, else the 8-byte entries (table_lds).  Grouped
 * launches and the decode kernels always use the 8-byte entries. */
#define RANS_F_TABLE8 8       /* always the 8-byte entries */
#define RANS_F_TABLE4 16      /* always the 4-byte entries: needs table_lds4 (else
                                 RANS_EARG) and S = 1 (else RANS_EUNSUPPORTED) */

typedef struct rans_w64_matrix {
    int32_t rows, cols;       /* out_features, and the stored columns: in_features,
                                 or in_features + 32 when in_features is an odd
                                 multiple of 32 (x rows then hold cols values, the
                                 last 32 zero; step's last 32 are zero) */
    int32_t R, C, S;          /* tile rows, tile columns, states per lane */
    int32_t max_tile_words;   /* largest tile block, in 16-bit words */
    int32_t max_state_words;  /* longest state stream (to the next state's start, the
                                 last state of a tile to the end of its padded block) */
    int32_t flags;            /* RANS_F_* launch options, 0 for the defaults */
    const uint16_t* words;    /* [tile_off[ntiles]] */
    const uint32_t* tile_off; /* [ntiles+1], in words, multiples of 8 */
    const uint8_t* slen;      /* [ntiles*64*S], length delta | state exponent << 4 */
    const uint32_t* tile_meta;/* [ntiles], length base | blob words << 16 */
    const uint32_t* table;    /* [4096], reference packing (host decoder) */
    const uint32_t* table_lds;/* [8192], the table as the kernels hold it in LDS, made
                                 by rans_table_lds from table (device kernels) */
    const int32_t* esc_tileptr;/* [ntiles+1] */
    const uint16_t* esc_pos;  /* [nesc], tile column * R + tile row */
    const int16_t* esc_val;   /* [nesc], the escaped codes */
    const float* step;        /* [cols] per-column step (waterfilling) */
    void* workspace;          /* split-K partials + counters; zero-filled once */
    int64_t workspace_bytes;
    const uint32_t* table_lds4;/* [4096] or NULL: the table as 4-byte LDS entries, made by
                                 rans_table_lds4 (GEMV only; see RANS_F_TABLE4) */
} rans_w64_matrix;

/* ---------------------------------------------------------------- device */

/* Fused decode + GEMV: y[b, r] = sum_c code[r,c] * (x[b,c] * step[c]) for
 * b < batch.  x is batch x cols (f32 or bf16, RANS_X_*), y is batch x rows
 * f32, written (never accumulated into).  The per-column step is folded into
 * x inside the kernel.  Replaces launch_rans_gemv (rans_gemv.cu:146-153),
 * which takes a host-folded f32 x and needs y zeroed when cols != C. */
int rans_w64_gemv(const rans_w64_matrix* m, const void* x, int x_dtype, int batch,
                  void* y, hipStream_t stream);

/* 1 when rans_w64_gemv at this batch and x dtype would run any of its
 * launches with the 4-byte table entries, were table_lds4 set (0 if not, or
 * a negative RANS_E* for arguments it would reject).  A caller asks before
 * building the 16 KB image, which only such matrices need.  Uses the
 * current device's occupancy figures; launches nothing.  No reference
 * counterpart. */
int rans_gemv_table4(const rans_w64_matrix* m, int x_dtype, int batch);

/* Bytes of workspace rans_w64_gemv needs for this matrix and batch (0 when
 * one workgroup covers a whole tile row).  The first 4096 bytes are counters
 * that must be zero before the first launch; the kernel leaves them zero. */
int64_t rans_gemv_workspace_bytes(const rans_w64_matrix* m, int batch);

/* 1 when a single-matrix rans_w64_gemv launch at this batch and x dtype would
 * take two tile rows per workgroup (one staged table serving both rows'
 * waves), 0 if not, or a negative RANS_E* for arguments it would reject.
 * Uses the current device's CU count; launches nothing.  No reference
 * counterpart. */
int rans_gemv_rows2(const rans_w64_matrix* m, int x_dtype, int batch);

/* rans_w64_gemv without a workspace, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No reference counterpart.  The same
 * kernels and the same results, bit for bit; m->workspace is ignored: the
 * split-K partial sums and arrival counters live in a file-scope device
 * array of RANS_SCRATCH_BYTES per GPU, held until the process ends.  Calls
 * no allocating routine.  The first call on a device looks the array up and
 * clears its counters with a fill kernel on `stream`; every launch leaves
 * them at zero.  Every call on one GPU shares that GPU's array, so calls
 * that overlap on one GPU (two streams, or two host threads) race: the
 * caller serialises them.  Returns RANS_ESCRATCH, before touching the
 * device, when the launch needs more than 16384 tile rows of counters or
 * more partials than the array holds. */
int rans_w64_gemv_noalloc(const rans_w64_matrix* m, const void* x, int x_dtype, int batch,
                          void* y, hipStream_t stream);

/* rans_w64_gemv for n <= 4 matrices that share x, in one launch:
 * ys[i] (batch x ms[i]->rows f32) gets ms[i]'s product.  No reference
 * counterpart: it is for projections that read the same activations (a
 * layer's q, k and v, or its gate and up), whose separate GEMVs each leave
 * most of the chip idle.  The matrices must have the same cols, R and S = 1,
 * and one workgroup per tile row (cols/C equal to the waves per workgroup,
 * the same for all: cols/C <= 8 and the tile block within LDS); otherwise
 * RANS_EUNSUPPORTED (or RANS_EGEOMETRY) and nothing is launched.  Results
 * are bitwise those of separate rans_w64_gemv calls. */
int rans_w64_gemv_group(const rans_w64_matrix* const* ms, int n, const void* x, int x_dtype,
                        int batch, float* const* ys, hipStream_t stream);

/* Decode to a dense bf16 matrix out[r,c] = bf16(code[r,c]*step[c]) (round to
 * nearest even).  Replaces launch_rans_decode (rans_gemv.cu:155-162). */
int rans_w64_decode(const rans_w64_matrix* m, void* out_bf16, hipStream_t stream);

/* Decode to dense int32 codes out[r,c] = code[r,c], escapes included: the
 * bit-exact check path.  No reference counterpart (the reference compares
 * the bf16 decode, bench.py:49-51). */
int rans_w64_decode_codes(const rans_w64_matrix* m, int32_t* out, hipStream_t stream);

/* Fixed-rate 4-bit baseline GEMV, same contract as the reference
 * (rans_gemv.cu:164-170): w packs 8 codes per u32 (nibble b of word j of row
 * r is column 8j+b, value nibble-8), x is the host-folded f32 x*step, y f32.
 * cols % 32 == 0 and w, x 16-byte aligned, else RANS_EGEOMETRY. */
int launch_int4_gemv(const void* w, const void* x, void* y, int rows, int cols,
                     hipStream_t stream);

/* Dense bf16 GEMV comparator: y[r] = sum_c W[r,c] * x[c] with W rows x cols
 * bf16 row-major, x bf16, y f32 (f32 accumulation).  The reference times this
 * product through torch's F.linear (bench.py:96); this is the uncompressed
 * HBM-bound GEMV written like the others here, so the compressed kernels are
 * also compared against a bf16 GEMV that runs near the HBM bound.  cols % 8
 * == 0 and w, x 16-byte aligned, else RANS_EGEOMETRY; RANS_EARG for null
 * pointers or non-positive sizes. */
int bf16_gemv(const void* w, const void* x, void* y, int rows, int cols, hipStream_t stream);

/* The reference's two rANS entry points, with its argument lists and stream
 * format (rans_gemv.cu:146-162, bound by kernel/rans.py:25-29 as
 * [c_int] + [c_void_p]*5 + [c_int]*3 + [c_void_p]): words / offs / table as
 * the reference's encode returns them (kernel/rans.py:62-98, 32-lane tiles of
 * R x C, R in {1, 2, 4, 8, 16}, C % 32 == 0, codes in [-128, 127]).
 * launch_rans_gemv: y[r] = sum_c code[r,c] * x[c] for the host-folded f32
 * x = x*step, written when cols == C, else added into y, which the caller
 * zeroes (rans.py:141-146).  launch_rans_decode: out[r,c] = bf16(code[r,c] *
 * step[c]).  Another R returns RANS_EUNSUPPORTED (-1, the reference's own
 * code) before anything is touched; RANS_EARG / RANS_EGEOMETRY for null
 * pointers or a shape that does not divide.  `words` must be device memory of
 * one allocation (hipMemGetAddressRange finds its end; no read goes past
 * it).  The format's streams are few and long, so this is the compatibility
 * path: rans_w64_gemv on the w64 layout is the fast one. */
int launch_rans_gemv(int R, const void* words, const void* offs, const void* table,
                     const void* x, void* y, int rows, int cols, int C, hipStream_t stream);
int launch_rans_decode(int R, const void* words, const void* offs, const void* table,
                       const void* step, void* out_bf16, int rows, int cols, int C,
                       hipStream_t stream);

/* ------------------------------------------------------------------ host */

/* Static 12-bit table from a symbol histogram, rans.py:34-51: freq[256],
 * cum[256], table[4096].  Returns RANS_ECODES for an empty or single-symbol
 * distribution. */
int rans_build_table(const uint8_t* sym, int64_t n, int64_t* freq, int64_t* cum,
                     uint32_t* table);

/* The LDS image of a reference-packed table: out[2*slot] = freq | code<<24
 * (code = sym-128, and 0 for the escape symbol 0, whose value comes from the
 * side table), out[2*slot+1] = slot - cum.  The device kernels copy these
 * 32 KB into LDS verbatim.  No reference counterpart: the reference unpacks
 * the fields on every symbol (rans_gemv.cu:33-36).  Returns RANS_EARG for a
 * null pointer. */
int rans_table_lds(const uint32_t* table, uint32_t* out);

/* The 4-byte LDS image: out[slot] = freq | (slot-cum)<<12 | code<<24 (code as
 * in rans_table_lds), 16 KB.  No reference counterpart.  Returns RANS_EARG
 * for a null pointer. */
int rans_table_lds4(const uint32_t* table, uint32_t* out);

/* Encode int32 codes (rows x cols, row-major) into the w64 format; replaces
 * encode() (rans.py:62-98).  R*C <= 65536 (the side table's 16-bit
 * positions), else RANS_EGEOMETRY; RANS_ECODES for a code outside
 * [-32768, 32767] (the side table's 16-bit values); RANS_ETILE when a tile block
 * exceeds 65535 words or a tile's length base 255 words.  On success *handle
 * owns the result and info[]
 * receives {nwords, ntiles, nstates, nesc, max_tile_words, payload_words,
 * max_state_words}.
 * Fetch the arrays with rans_w64_encode_fetch, then free the handle. */
int rans_w64_encode(const int32_t* codes, int32_t rows, int32_t cols, int32_t R, int32_t C,
                    int32_t S, int32_t nthreads, void** handle, int64_t* info);

int rans_w64_encode_fetch(void* handle, uint16_t* words, uint32_t* tile_off,
                          uint32_t* tile_meta, uint8_t* slen, uint32_t* table, int64_t* freq,
                          int32_t* esc_tileptr, uint16_t* esc_pos, int16_t* esc_val);

/* The symbol counts over the encoded matrix (256 x int64, symbol = code+128,
 * 0 for escapes), for the bit accounting.  No reference counterpart (the
 * reference recounts with numpy, rans.py:95-97). */
int rans_w64_encode_counts(void* handle, int64_t* counts);

void rans_w64_encode_free(void* handle);

/* Host decoder of the w64 format to int32 codes (escapes applied); replaces
 * decode_ref (rans.py:101-123).  Returns state+1 (positive) for the first
 * state whose final value is not 2^16 (the reference's final-state assert,
 * rans.py:121), RANS_EARG on a stream overrun, a stream read to other than
 * its stored length (short only where padded to its tile's base), or an
 * escape side table that disagrees with the escape symbols in the stream. */
int rans_w64_decode_host(const rans_w64_matrix* m_host, int32_t* out);

/* The reference's encoder for its own 32-lane layout (kernel/rans.py:62-98),
 * the input of launch_rans_gemv / launch_rans_decode: codes (rows x cols,
 * int32 in [-128, 127], else RANS_ECODES) in R x C tiles (C % 32 == 0);
 * writes words (capacity words_cap >= 2*lanes + rows*cols + 8, lanes =
 * 32*(rows/R)*(cols/C)), offs[lanes] and table[4096] exactly as the
 * reference's encode lays them out, and info[0] = words used (with the 8
 * trailing zero words), info[1] = renormalisation words.  Host only. */
int rans_ref32_encode(const int32_t* codes, int32_t rows, int32_t cols, int32_t R, int32_t C,
                      int32_t nthreads, uint16_t* words, int64_t words_cap, uint32_t* offs,
                      uint32_t* table, int64_t* info);

#ifdef __cplusplus
}
#endif

#endif /* VRAMC_RANS_H */
