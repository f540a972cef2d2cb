/*
 * oracle/fir_oracle.c -- CPU restatement of the causal K-tap FIR contract.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker for the HIP FIR kernels.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * the library built from it; the product path never does.
 *
 * Contract (restates /root/reference/src/triton_pnfirtau.py:40-135):
 *   taps are fp32, stored oldest-lag first: taps[K-1] is lag 0 (the present row),
 *   taps[0] is lag K-1 (src/pnfirtau_attention.py:56, triton_pnfirtau.py:62-69).
 *   forward  y[n] = x[n]*h0, then acc = fmaf(x[n-u], h_u, acc) for u = 1..K-1 while n-u >= 0
 *            (triton_pnfirtau.py:72-84; Triton's default fp-fusion turns `acc += a*b`
 *            into one fused multiply-add).
 *   backward gx[n] = gy[n]*h0, then acc = fmaf(gy[n+u], h_u, acc) while n+u < N
 *            (triton_pnfirtau.py:120-132).
 *   The fp32 accumulator is rounded once to the storage type (RNE for bf16).
 *
 * Layout: contiguous [BH, N, C]; taps [G, K] with G == 1 (shared) or G == H
 * (per-head: the tap row of slice bh is bh % G).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static float bf16_bits_to_f32(uint16_t h) {
    uint32_t u = ((uint32_t)h) << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static uint16_t f32_to_bf16_bits_rne(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) {
        return (uint16_t)((u >> 16) | 0x0040u); /* quiet NaN */
    }
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

static float fir_point(const float* col, int64_t n, int64_t N, int64_t stride,
                       const float* taps, int K, int adjoint) {
    float acc = col[n * stride] * taps[K - 1];
    for (int u = 1; u < K; ++u) {
        int64_t m = adjoint ? n + u : n - u;
        if (m < 0 || m >= N) break;
        acc = fmaf(col[m * stride], taps[K - 1 - u], acc);
    }
    return acc;
}

/* fp32 in, fp32 out. */
void oracle_fir_f32(const float* x, float* y, int64_t BH, int64_t N, int64_t C,
                    const float* taps, int64_t G, int K, int adjoint) {
    for (int64_t bh = 0; bh < BH; ++bh) {
        const float* t = taps + (bh % G) * K;
        for (int64_t c = 0; c < C; ++c) {
            const float* col = x + bh * N * C + c;
            for (int64_t n = 0; n < N; ++n) {
                y[bh * N * C + n * C + c] = fir_point(col, n, N, C, t, K, adjoint);
            }
        }
    }
}

/* bf16 bits in, bf16 bits out (RNE). */
void oracle_fir_bf16(const uint16_t* x, uint16_t* y, int64_t BH, int64_t N, int64_t C,
                     const float* taps, int64_t G, int K, int adjoint) {
    float buf[4096];
    for (int64_t bh = 0; bh < BH; ++bh) {
        const float* t = taps + (bh % G) * K;
        for (int64_t c = 0; c < C; ++c) {
            for (int64_t n0 = 0; n0 < N; n0 += 4096 - 64) {
                /* stage a window of one channel column (with a K-row halo) in fp32 */
                int64_t lo = adjoint ? n0 : (n0 - (K - 1) < 0 ? 0 : n0 - (K - 1));
                int64_t hi_out = n0 + (4096 - 64) < N ? n0 + (4096 - 64) : N;
                int64_t hi = adjoint ? (hi_out + (K - 1) < N ? hi_out + (K - 1) : N) : hi_out;
                for (int64_t m = lo; m < hi; ++m)
                    buf[m - lo] = bf16_bits_to_f32(x[bh * N * C + m * C + c]);
                for (int64_t n = n0; n < hi_out; ++n) {
                    float acc = buf[n - lo] * t[K - 1];
                    for (int u = 1; u < K; ++u) {
                        int64_t m = adjoint ? n + u : n - u;
                        if (m < 0 || m >= N) break;
                        acc = fmaf(buf[m - lo], t[K - 1 - u], acc);
                    }
                    y[bh * N * C + n * C + c] = f32_to_bf16_bits_rne(acc);
                }
            }
        }
    }
}
