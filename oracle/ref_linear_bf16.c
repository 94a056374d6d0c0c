/* ref_linear_bf16.c -- CPU baseline, not a checker: a C restatement of the
 * reference's own CPU Linear::forward on a BF16 weight (the path the
 * reference's published CPU timings measure), step for step and at the same
 * cost, so that bench.py can time it on the host beside the GPU path.
 * Test infrastructure like the rest of oracle/: only tests/ and bench.py's
 * CPU baseline call it.
 *
 * lluda-inference, CPU build (no "gpu" feature):
 *   Linear::forward            src/attention.rs:101-136
 *     x.reshape([m, k])        src/tensor.rs:385-404    (copies the data)
 *     weight.transpose()       src/tensor.rs:439-467    (a new [k][n] BF16 buffer, every call)
 *     x_2d.matmul(&weight_t)   src/tensor.rs:804-818, 945-958
 *       to_vec_f32() of both   src/tensor.rs:312-321    (a clone of x; BF16 -> F32 of the weight,
 *                                                        src/bf16.rs:79-81, 136-142)
 *       matmul_2d              src/tensor.rs:2716-2753  (naive i, j, k loops, f32 sum += a * b)
 *     output reshape           src/tensor.rs:385-404    (copies the data)
 * Built with -ffp-contract=off: Rust does not fuse a * b + c. */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static float bf16_to_f32(uint16_t h) {
    const uint32_t bits = (uint32_t)h << 16;
    float f;
    memcpy(&f, &bits, sizeof f);
    return f;
}

/* y[m][n_out] = x[m][k_in] . w[n_out][k_in]^T.  Returns 0, or -1 when an
 * allocation fails (y untouched). */
int ref_linear_forward_bf16(const uint16_t* w, size_t n_out, size_t k_in, const float* x, size_t m, float* y) {
    const size_t n = n_out, k = k_in;
    float* x2 = malloc(m * k * sizeof(float));          /* reshape copy */
    uint16_t* wt = malloc(k * n * sizeof(uint16_t));    /* transposed BF16 weight */
    float* lhs = malloc(m * k * sizeof(float));         /* to_vec_f32 of x_2d */
    float* rhs = malloc(k * n * sizeof(float));         /* to_vec_f32 of weight_t */
    float* out = malloc(m * n * sizeof(float));         /* matmul_2d result */
    if (!x2 || !wt || !lhs || !rhs || !out) {
        free(x2); free(wt); free(lhs); free(rhs); free(out);
        return -1;
    }
    memcpy(x2, x, m * k * sizeof(float));
    /* transpose: input [n][k] -> output [k][n], output[j * n + i] = input[i * k + j] */
    for (size_t i = 0; i < n; i++)
        for (size_t j = 0; j < k; j++) wt[j * n + i] = w[i * k + j];
    memcpy(lhs, x2, m * k * sizeof(float));
    for (size_t i = 0; i < k * n; i++) rhs[i] = bf16_to_f32(wt[i]);
    for (size_t i = 0; i < m; i++)
        for (size_t j = 0; j < n; j++) {
            float sum = 0.0f;
            for (size_t kk = 0; kk < k; kk++) sum += lhs[i * k + kk] * rhs[kk * n + j];
            out[i * n + j] = sum;
        }
    memcpy(y, out, m * n * sizeof(float)); /* output reshape copy */
    free(x2); free(wt); free(lhs); free(rhs); free(out);
    return 0;
}
