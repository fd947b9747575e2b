// Host build of the K-quant layout code of the device header (Q3K::pack_unit,
// Q3K::unit_parts, Q3K::words, Q3KSB::pack/unpack, sb_geom/sb_piece: the same source the repack, verify and matvec kernels
// compile) checked against the oracle on seeded GGUF rows:
//  * unit_parts(pack_unit(g)) returns every value's low 2 bits and high bit;
//  * the per-16 integer dots formed from words() (the matvec's assembly, each
//    sub-block's dot started from -4 * GS * sum(x)) equal GS times the
//    oracle's uqo_q3k_block_dots;
//  * the row sum d*xs0*(s0*D0 + s1*D1) + d*(xs1/16)*(s2*D2 + s3*D3) over the
//    units, with the scales and d read from the packed words, rounds to the
//    oracle's uqo_matvec_x output within 1 ulp;
//  * every unit word above is taken after a round trip through the row-block
//    pieces (Q3KSB::pack, then Q3KSB::unpack), which returns the words exactly;
//  * sb_geom / sb_piece place every piece of every superblock of a weight at
//    a distinct 16-byte slot inside blocks * LB * P * 16 bytes.
// Exit status 0 when every check holds.
#include "../uefi-gpu_amd/csrc/uq_units.h"
#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

extern "C" {
void uqo_quant_act(const float* x, int64_t n, float* scale, int8_t* q);
void uqo_q3k_block_dots(const uint8_t* w, int64_t n, int64_t m, const int8_t* qx, int32_t* dots);
void uqo_matvec_x(uint32_t kind, const uint8_t* w, int64_t n, int64_t m, const float* x, float* y);
float uqo_half(uint16_t h);
}

static int dot4(int a, int b, int c) {
    for (int k = 0; k < 4; k++) c += (int)(int8_t)(a >> (8 * k)) * (int)(int8_t)(b >> (8 * k));
    return c;
}

int main() {
    std::mt19937 rng(0x5EED0003u);
    long bad_parts = 0, bad_dots = 0, bad_rows = 0, rows_total = 0, bad_sb = 0, bad_geom = 0;
    // row-block geometry: pieces of distinct (row, superblock, piece) land on
    // distinct slots inside the allocation
    for (int n : {256, 768, 1536, 2048, 3072, 6144, 8960, 16384}) {
        for (int m : {1, 7, 10, 11, 100}) {
            const uq::SbGeom g = uq::sb_geom(n, m);
            // whole waves, at least one row, and no block size of 1-4 waves
            // with a smaller share of idle slots
            bool worse = false;
            for (int lb = 64; lb <= 256; lb += 64) {
                const int rb = lb / (n / 256);
                if (rb >= 1 && (int64_t)(lb - rb * g.S) * g.LB < (int64_t)(g.LB - g.RB * g.S) * lb) worse = true;
            }
            if (!g.LB || g.LB % 64 || g.LB > 256 || g.RB * g.S > g.LB || g.RB < 1 || worse) {
                bad_geom++;
                continue;
            }
            for (int P : {7}) {
                const int64_t slots = g.blocks * g.LB * P;
                std::vector<char> seen((size_t)slots, 0);
                for (int r = 0; r < m; r++)
                    for (int sb = 0; sb < g.S; sb++)
                        for (int k = 0; k < P; k++) {
                            const int64_t o = uq::sb_piece(r, sb, k, g.S, g.LB, g.RB, P);
                            if (o % 16 || o < 0 || o / 16 >= slots || seen[(size_t)(o / 16)]++) bad_geom++;
                        }
            }
        }
    }
    for (int n : {256, 768, 1536, 2048}) {
        const int m = 24, nsb = n / 256;
        std::vector<uint8_t> w((size_t)m * nsb * 110);
        for (auto& b : w) b = (uint8_t)(rng() & 255);
        for (int i = 0; i < m * nsb; i++) {  // finite d, |d| < 2^-6
            const uint16_t d = (uint16_t)((rng() & 0x83ff) | (0x1000 + (rng() % 0x0c00)));
            w[(size_t)i * 110 + 108] = (uint8_t)d;
            w[(size_t)i * 110 + 109] = (uint8_t)(d >> 8);
        }
        std::vector<float> x(n), xs(n / 32), y(m);
        std::normal_distribution<float> nd(0.0f, 1.0f);
        for (auto& v : x) v = nd(rng);
        if (n == 768) for (int k = 0; k < 64; k++) x[k] = (k & 1) ? 127.0f : -127.0f;  // amax blocks
        std::vector<int8_t> qx(n);
        uqo_quant_act(x.data(), n, xs.data(), qx.data());
        std::vector<int32_t> dots((size_t)m * (n / 16));
        uqo_q3k_block_dots(w.data(), n, m, qx.data(), dots.data());
        uqo_matvec_x(11u, w.data(), n, m, x.data(), y.data());
        for (int r = 0; r < m; r++) {
            double acc = 0.0;
            for (int sb = 0; sb < nsb; sb++) {
                const uint8_t* g = w.data() + ((size_t)r * nsb + sb) * 110;
                uint32_t UA[4][4], UP[4][4], UA2[4][4], UP2[4][4], pw[28];
                for (int p = 0; p < 4; p++) uq::Q3K::pack_unit(g, p, UA[p], UP[p]);
                uq::Q3KSB::pack(UA, UP, pw);
                uq::Q3KSB::unpack(pw, UA2, UP2);
                bad_sb += std::memcmp(UA, UA2, sizeof(UA)) != 0 || std::memcmp(UP, UP2, sizeof(UP)) != 0;
                for (int p = 0; p < 4; p++) {
                    const uint32_t* A = UA2[p];
                    const uint32_t* P = UP2[p];
                    for (int c = 0; c < 4; c++)
                        for (int t = 0; t < 4; t++)
                            for (int b = 0; b < 4; b++) {
                                int l2, hb;
                                uq::Q3K::unit_parts(A, P, c, t, b, l2, hb);
                                const int i = 64 * p + 16 * c + 4 * t + b;
                                bad_parts += l2 != uq::Q3K::gguf_low2(g, i) || hb != uq::Q3K::gguf_hbit(g, i);
                            }
                    const int u = 4 * sb + p;
                    const int8_t* xu = qx.data() + 64 * u;
                    int D[4];
                    for (int c = 0; c < 4; c++) {
                        int sum = 0;
                        for (int l = 0; l < 16; l++) sum += xu[16 * c + l];
                        D[c] = sum * (c >= 2 ? -64 : -4);
                    }
                    for (int t = 0; t < 4; t++) {
                        int wd[4];
                        uq::Q3K::words(A[t], t < 2 ? P[0] : P[1], t, wd);
                        for (int c = 0; c < 4; c++) {
                            int xw;
                            std::memcpy(&xw, xu + 16 * c + 4 * t, 4);
                            D[c] = dot4(wd[c], xw, D[c]);
                        }
                    }
                    for (int c = 0; c < 4; c++)
                        bad_dots += D[c] != (c >= 2 ? 16 : 1) * dots[(size_t)r * (n / 16) + 4 * u + c];
                    const int sc = (int)P[2];
                    const int s0 = (int8_t)sc, s1 = (int8_t)(sc >> 8), s2 = (int8_t)(sc >> 16), s3 = sc >> 24;
                    const double dd = (double)uqo_half((uint16_t)P[3]);
                    const double T0 = (double)s0 * D[0] + (double)s1 * D[1], T1 = (double)s2 * D[2] + (double)s3 * D[3];
                    acc += (dd * (double)xs[2 * u]) * T0 + (dd * ((double)xs[2 * u + 1] / 16)) * T1;
                }
            }
            const float yf = (float)acc;
            uint32_t a, b;
            std::memcpy(&a, &yf, 4);
            std::memcpy(&b, &y[r], 4);
            const long diff = (long)a - (long)b;
            bad_rows += (diff > 1 || diff < -1) && !(yf == 0.0f && y[r] == 0.0f);
            rows_total++;
        }
    }
    printf("parts differing: %ld, dots differing: %ld, rows beyond 1 ulp: %ld of %ld\n", bad_parts, bad_dots,
           bad_rows, rows_total);
    printf("row-block round trips differing: %ld, geometry faults: %ld\n", bad_sb, bad_geom);
    return bad_parts || bad_dots || bad_rows || bad_sb || bad_geom;
}
