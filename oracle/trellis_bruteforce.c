/* Brute-force C restatement of the EXL3 trellis tile decode (mul1 codebook). TEST INFRASTRUCTURE ONLY.
 *
 * A second, independent statement of the tile format next to the vectorised NumPy oracle:
 *   - the tile's 256*K-bit ring is materialised bit by bit (bit b = bit 31 - b%32 of little-endian word b/32,
 *     ext-op-inventory.md:717-725), and every 16-bit window is read one bit at a time, wrapping around the ring
 *     (tail-biting; the window of position t ends at bit (t+1)K);
 *   - the position -> (row, col) map uses the ring form of dsv41/xpu/dsv_xpu/exl3_tri.py:4-9
 *     (t = i/8, j = i%8: r = (t%4)*2 + (j&1) + 8((j>>1)&1), c = t/4 + 8((j>>2)&1)), not the bit-field form the
 *     NumPy oracle uses (glm/xpu/csrc/exl3_esimd.h:7-8);
 *   - mul1 (glm/xpu/csrc/exl3_esimd.h:46-68): x = st * 0x83DCD12D mod 2^32, the byte sum by a loop, the affine in
 *     double, and a hand-written round-to-nearest-even double -> binary16 conversion (no compiler half type).
 */
#include <stdint.h>
#include <math.h>
#include <string.h>

/* round-to-nearest-even double -> IEEE binary16 bits; handles normals, subnormals, overflow to inf */
static uint16_t f64_to_f16_bits(double v) {
    uint16_t sign = 0;
    if (signbit(v)) { sign = 0x8000; v = -v; }
    if (v == 0.0) return sign;
    if (v >= 65520.0) return sign | 0x7C00;              /* rounds to inf */
    int e = 0;
    double m = v;
    while (m >= 2.0) { m /= 2.0; e++; }
    while (m < 1.0) { m *= 2.0; e--; }
    /* v = m * 2^e, 1 <= m < 2 */
    int exp16 = e + 15;
    double q;           /* value in units of the target lsb */
    if (exp16 >= 1) q = m * 1024.0;                       /* 10 fraction bits */
    else { q = v / (1.0 / 16777216.0); exp16 = 0; }      /* subnormal: lsb 2^-24 */
    double fl = (double)(int64_t)q;
    double fr = q - fl;
    int64_t r = (int64_t)fl;
    if (fr > 0.5 || (fr == 0.5 && (r & 1))) r++;
    if (exp16 >= 1) {
        if (r == 2048) { r = 1024; exp16++; }
        if (exp16 >= 31) return sign | 0x7C00;
        return sign | (uint16_t)(exp16 << 10) | (uint16_t)(r - 1024);
    }
    /* subnormal (r may round up to 1024 = smallest normal, which the bit pattern expresses naturally) */
    return sign | (uint16_t)r;
}

uint16_t exl3_bf_mul1(uint32_t state) {
    uint32_t x = (uint32_t)(state & 0xFFFFu) * 0x83DCD12Du;
    uint32_t s = 0;
    for (int i = 0; i < 4; ++i) s += (x >> (8 * i)) & 0xFFu;
    double h = 1024.0 + (double)s;
    return f64_to_f16_bits(h * 0.00676727294921875 - 10.3828125);
}

uint16_t exl3_bf_f64_to_f16(double v) { return f64_to_f16_bits(v); }

/* tile: 16K int16 values (one tile of a [k/16, n/16, 16K] trellis). out: 256 fp16 bit patterns, out[row*16+col]. */
int exl3_bf_decode_tile(const int16_t* tile, int K, uint16_t* out) {
    if (K < 1 || K > 8) return 1;
    const int nbits = 256 * K;
    const int nwords = 8 * K;
    uint32_t words[64];
    for (int i = 0; i < nwords; ++i)
        words[i] = (uint32_t)(uint16_t)tile[2 * i] | ((uint32_t)(uint16_t)tile[2 * i + 1] << 16);
    uint8_t bits[2048];
    for (int b = 0; b < nbits; ++b) bits[b] = (uint8_t)((words[b / 32] >> (31 - b % 32)) & 1u);
    for (int i = 0; i < 256; ++i) {
        uint32_t st = 0;
        int end = (i + 1) * K;
        for (int j = 0; j < 16; ++j) {
            int b = ((end - 16 + j) % nbits + nbits) % nbits;
            st = (st << 1) | bits[b];
        }
        int t = i / 8, jj = i % 8;
        int r = (t % 4) * 2 + (jj & 1) + 8 * ((jj >> 1) & 1);
        int c = t / 4 + 8 * ((jj >> 2) & 1);
        out[r * 16 + c] = exl3_bf_mul1(st);
    }
    return 0;
}

/* A whole trellis [tk, tn, 16K] -> fp16 bits [tk*16, tn*16] row-major (W_hat, Hadamard domain). */
int exl3_bf_reconstruct(const int16_t* trellis, int tk, int tn, int K, uint16_t* out) {
    uint16_t tile[256];
    for (int a = 0; a < tk; ++a)
        for (int b = 0; b < tn; ++b) {
            int rc = exl3_bf_decode_tile(trellis + ((int64_t)a * tn + b) * 16 * K, K, tile);
            if (rc) return rc;
            for (int r = 0; r < 16; ++r)
                for (int c = 0; c < 16; ++c)
                    out[((int64_t)a * 16 + r) * (tn * 16) + b * 16 + c] = tile[r * 16 + c];
        }
    return 0;
}
