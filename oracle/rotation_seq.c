/* CPU oracle: the reference's group-wise Hadamard rotation with the
 * reference's own fp32 rounding.  TEST INFRASTRUCTURE ONLY (see torch_ref.py).
 *
 * converter/rotation.py:82-92 rotates weights as `x @ H.T` and :237-248 the
 * Hessian as einsum("kp,nkl,le->npe", R, H, R).  Run by torch on the CPU, both
 * are fp32 GEMMs in which every output is one fused multiply-add chain over
 * the contraction index in increasing order, starting from zero; for a group
 * of 512 the sum is two 256-long chains added (tests/test_oracle.py checks
 * this restatement against the reference's own outputs,
 * tests/golden/golden_rotation.safetensors).  Written out here so the
 * oracle's rotation does not depend on the BLAS of the host it runs on.
 *
 * Hd[k][j] = m * (-1)^s(k, j): regular size 4^n: m = 2^-n, s = number of
 * base-4 digits with k_d + j_d = 3; Sylvester size 2^n: m = fp32(1/sqrt(2^n)),
 * s = popcount(k & j) (converter/rotation.py:26-62). */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>

static int is_pow4(int n) { return n >= 4 && (n & (n - 1)) == 0 && (n & 0x55555555) == n; }

static float* hd_table(int rot) {
    float* h = (float*)malloc(sizeof(float) * (size_t)rot * rot);
    if (!h) return NULL;
    const int reg = is_pow4(rot);
    float m = 1.0f;
    if (reg) {
        for (int r = rot; r > 1; r >>= 2) m *= 0.5f;
    } else {
        m = (float)(1.0 / sqrt((double)rot));
    }
    for (int k = 0; k < rot; ++k)
        for (int j = 0; j < rot; ++j) {
            unsigned t = (unsigned)(k ^ j);
            int s = reg ? __builtin_popcount(t & (t >> 1) & 0x55555555u) & 1 : __builtin_popcount((unsigned)(k & j)) & 1;
            h[(size_t)k * rot + j] = s ? -m : m;
        }
    return h;
}

/* y[r][g*rot + j] = chain_k x[r][g*rot + k] * Hd[k][j]  (x already padded,
 * [rows, cols] with cols % rot == 0).  rot: 2 .. 512.  Returns 0, or -1. */
int oracle_rotate_rows(const float* x, int64_t rows, int64_t cols, float* y, int rot, int threads) {
    if (rot < 2 || rot > 512 || (rot & (rot - 1)) || cols % rot) return -1;
    float* h = hd_table(rot);
    if (!h) return -1;
    const int kc = rot > 256 ? 256 : rot;
    const int64_t groups = cols / rot;
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int64_t rg = 0; rg < rows * groups; ++rg) {
        const float* xg = x + (rg / groups) * cols + (rg % groups) * rot;
        float* yg = y + (rg / groups) * cols + (rg % groups) * rot;
        float acc[512], part[512];
        for (int c = 0; c < rot; c += kc) {
            for (int j = 0; j < rot; ++j) acc[j] = 0.0f;
            for (int k = c; k < c + kc; ++k) {
                const float xk = xg[k];
                const float* hk = h + (size_t)k * rot;
                for (int j = 0; j < rot; ++j) acc[j] = fmaf(xk, hk[j], acc[j]);
            }
            for (int j = 0; j < rot; ++j) part[j] = c ? part[j] + acc[j] : acc[j];
        }
        for (int j = 0; j < rot; ++j) yg[j] = part[j];
    }
    free(h);
    return 0;
}

/* out[b] = (Hd^T blk[b]) Hd for `nb` blocks [rot, rot]: the left product as
 * chains over the block's rows, then the right product as chains over the
 * intermediate's columns.  rot: a power of 4 up to 256. */
int oracle_rotate_blocks(const float* blk, int64_t nb, float* out, int rot, int threads) {
    if (!is_pow4(rot) || rot > 256) return -1;
    float* h = hd_table(rot);
    if (!h) return -1;
    int err = 0;
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int64_t b = 0; b < nb; ++b) {
        const float* B = blk + b * (int64_t)rot * rot;
        float* O = out + b * (int64_t)rot * rot;
        float* T = (float*)malloc(sizeof(float) * (size_t)rot * rot);
        if (!T) {
            err = 1;
            continue;
        }
        /* T[p][l] = chain_k Hd[k][p] B[k][l]: row p of T accumulates rows k of B */
        for (int p = 0; p < rot; ++p) {
            float* tp = T + (size_t)p * rot;
            for (int l = 0; l < rot; ++l) tp[l] = 0.0f;
            for (int k = 0; k < rot; ++k) {
                const float hkp = h[(size_t)k * rot + p];
                const float* bk = B + (size_t)k * rot;
                for (int l = 0; l < rot; ++l) tp[l] = fmaf(hkp, bk[l], tp[l]);
            }
        }
        /* O[p][e] = chain_l T[p][l] Hd[l][e] */
        for (int p = 0; p < rot; ++p) {
            float* op = O + (size_t)p * rot;
            const float* tp = T + (size_t)p * rot;
            for (int e = 0; e < rot; ++e) op[e] = 0.0f;
            for (int l = 0; l < rot; ++l) {
                const float tpl = tp[l];
                const float* hl = h + (size_t)l * rot;
                for (int e = 0; e < rot; ++e) op[e] = fmaf(tpl, hl[e], op[e]);
            }
        }
        free(T);
    }
    free(h);
    return err ? -1 : 0;
}
