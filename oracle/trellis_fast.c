/* Fast C restatement of the EXL3 trellis decode, for parity checks at full layer sizes. TEST INFRASTRUCTURE ONLY.
 *
 * A third statement of the decode next to the NumPy oracle and the bit-by-bit decoder of trellis_bruteforce.c, written
 * for speed (the NumPy form takes ~170 ns per weight): per position the window of the vector form of
 * ext-op-inventory.md:746-757 (ih = ((t+1)K - 1) / 32, il = ih - 1 mod 8K, state = (w[il] w[ih]) >> sh, 16 bits),
 * the codebook as a 65536-entry table filled by the brute-force statement (exl3_bf_mul1), and the bit-field position
 * map of glm/xpu/csrc/exl3_esimd.h:7-8. Tile-rows are split over OpenMP threads. tests/test_oracle.py pins it bit for
 * bit against the brute-force decoder and the NumPy oracle for K = 1..8, uniform and per-tile.
 */
#include <math.h>
#include <stdint.h>

uint16_t exl3_bf_mul1(uint32_t state);

static uint16_t g_lut[65536];     /* codebook, fp16 bits */
static double g_lutd[65536];      /* the same values as doubles */
static int g_lut_ok = 0;

/* IEEE binary16 bits -> double (finite values: the codebook has no inf / nan) */
static double f16_bits_to_double(uint16_t h) {
    const int e = (h >> 10) & 31, f = h & 1023;
    const double v = e ? ldexp(1024.0 + f, e - 25) : ldexp((double)f, -24);
    return (h & 0x8000) ? -v : v;
}

/* per K (1..8) and position t: the two words and the shift of the vector window form, and the tile cell row*16+col */
static uint8_t g_il[9][256], g_ih[9][256], g_sh[9][256], g_cell[256];

static void build_lut(void) {
    if (g_lut_ok) return;
    for (uint32_t s = 0; s < 65536u; ++s) {
        g_lut[s] = exl3_bf_mul1(s);
        g_lutd[s] = f16_bits_to_double(g_lut[s]);
    }
    for (int K = 1; K <= 8; ++K)
        for (int t = 0; t < 256; ++t) {
            const int W = 8 * K, e = (t + 1) * K, ih = (e - 1) / 32;
            g_ih[K][t] = (uint8_t)ih;
            g_il[K][t] = (uint8_t)((ih - 1 + W) % W);
            g_sh[K][t] = (uint8_t)(32 * (ih + 1) - e);
        }
    for (int t = 0; t < 256; ++t)
        g_cell[t] = (uint8_t)((8 * ((t >> 1) & 1) + 2 * ((t >> 3) & 3) + (t & 1)) * 16 + (t >> 5) + 8 * ((t >> 2) & 1));
    g_lut_ok = 1;
}

/* 16-bit state of position t of a tile (8K little-endian words): ih = ((t+1)K - 1) / 32, il = ih - 1 mod 8K,
 * sh = 32 (ih + 1) - (t+1)K, state = ((w[il] << 32) | w[ih]) >> sh (the tables above hold il, ih, sh) */
static inline uint32_t tile_state(const uint32_t* w, int K, int t) {
    return (uint32_t)(((((uint64_t)w[g_il[K][t]]) << 32) | (uint64_t)w[g_ih[K][t]]) >> g_sh[K][t]) & 0xFFFFu;
}

/* One tile into out[row * ld + col] (fp16 bits). */
static void decode_tile(const uint32_t* w, int K, uint16_t* out, int64_t ld) {
    for (int t = 0; t < 256; ++t) out[(g_cell[t] >> 4) * ld + (g_cell[t] & 15)] = g_lut[tile_state(w, K, t)];
}

/* trellis int16 [tk][tn][16K] -> fp16 bits [tk * 16][nts * 16] = W_hat[:, 16 n0t : 16 (n0t + nts)]. */
int exl3_fast_reconstruct(const int16_t* trellis, int64_t tk, int64_t tn, int K, int64_t n0t, int64_t nts,
                          uint16_t* out, int nthreads) {
    if (K < 1 || K > 8 || n0t < 0 || nts < 0 || n0t + nts > tn) return 1;
    build_lut();
    const uint32_t* words = (const uint32_t*)trellis;
    const int64_t ld = nts * 16;
#pragma omp parallel for schedule(static) num_threads(nthreads > 0 ? nthreads : 1)
    for (int64_t a = 0; a < tk; ++a)
        for (int64_t b = 0; b < nts; ++b)
            decode_tile(words + (a * tn + n0t + b) * 8 * K, K, out + a * 16 * ld + b * 16, ld);
    return 0;
}

/* Per-tile K: tile i (row-major over [tk][tn]) holds 8 kmap[i] words at words + woff[i]. out fp16 bits
 * [tk * 16][tn * 16]. */
int exl3_fast_reconstruct_mixed(const uint32_t* words, const uint8_t* kmap, const int64_t* woff, int64_t tk,
                                int64_t tn, uint16_t* out, int nthreads) {
    build_lut();
    int bad = 0;
    for (int64_t i = 0; i < tk * tn; ++i) bad |= kmap[i] < 1 || kmap[i] > 8;
    if (bad) return 1;
    const int64_t ld = tn * 16;
#pragma omp parallel for schedule(static) num_threads(nthreads > 0 ? nthreads : 1)
    for (int64_t a = 0; a < tk; ++a)
        for (int64_t b = 0; b < tn; ++b) {
            const int64_t i = a * tn + b;
            decode_tile(words + woff[i], kmap[i], out + a * 16 * ld + b * 16, ld);
        }
    return 0;
}

/* y[m][c] = sum_k x[m][k] * W_hat[k][c] in float64 for x float64 [m][16 tk] and W_hat the decoded trellis (uniform K:
 * `trellis` [tk][tn][16K]; per-tile K: `words`/`kmap`/`woff` with trellis NULL), without materialising W_hat: threads
 * own 16-column tile columns, and every column sums over k in order (tile-row by tile-row, row by row). y float64
 * [m][16 tn]. */
static void matmul_tiles(const int16_t* trellis, int K, const uint32_t* words, const uint8_t* kmap,
                         const int64_t* woff, int64_t tk, int64_t tn, const double* x, int64_t m, double* y,
                         int nthreads) {
    const int64_t k = tk * 16, n = tn * 16;
#pragma omp parallel for schedule(dynamic, 4) num_threads(nthreads > 0 ? nthreads : 1)
    for (int64_t b = 0; b < tn; ++b) {
        double w[16][16];        /* decoded tile [row][column] */
        double acc[16][16];      /* [row of x (16 at a time)][column] */
        for (int64_t m0 = 0; m0 < m; m0 += 16) {
            const int64_t mm = m - m0 < 16 ? m - m0 : 16;
            for (int64_t i = 0; i < mm; ++i)
                for (int c = 0; c < 16; ++c) acc[i][c] = 0.0;
            for (int64_t a = 0; a < tk; ++a) {
                const int64_t ti = a * tn + b;
                const uint32_t* tw = trellis ? (const uint32_t*)trellis + ti * 8 * K : words + woff[ti];
                const int Kt = trellis ? K : kmap[ti];
                double* wf = &w[0][0];
                for (int t = 0; t < 256; ++t) wf[g_cell[t]] = g_lutd[tile_state(tw, Kt, t)];
                for (int64_t i = 0; i < mm; ++i) {
                    const double* xr = x + (m0 + i) * k + a * 16;
                    for (int r = 0; r < 16; ++r) {
                        const double xv = xr[r];
                        for (int c = 0; c < 16; ++c) acc[i][c] += xv * w[r][c];
                    }
                }
            }
            for (int64_t i = 0; i < mm; ++i)
                for (int c = 0; c < 16; ++c) y[(m0 + i) * n + b * 16 + c] = acc[i][c];
        }
    }
}

int exl3_fast_matmul(const int16_t* trellis, int64_t tk, int64_t tn, int K, const double* x, int64_t m, double* y,
                     int nthreads) {
    if (K < 1 || K > 8) return 1;
    build_lut();
    matmul_tiles(trellis, K, 0, 0, 0, tk, tn, x, m, y, nthreads);
    return 0;
}

int exl3_fast_matmul_mixed(const uint32_t* words, const uint8_t* kmap, const int64_t* woff, int64_t tk, int64_t tn,
                           const double* x, int64_t m, double* y, int nthreads) {
    build_lut();
    int bad = 0;
    for (int64_t i = 0; i < tk * tn; ++i) bad |= kmap[i] < 1 || kmap[i] > 8;
    if (bad) return 1;
    matmul_tiles(0, 0, words, kmap, woff, tk, tn, x, m, y, nthreads);
    return 0;
}
