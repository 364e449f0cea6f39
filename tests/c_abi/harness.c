/*
 * harness.c -- the C ABI driven from plain C (C99, no Python, no torch), the
 * way a foreign-function binding such as JLUST's ccall reaches the library.
 * Device memory comes from the HIP runtime; every operand is a raw device
 * pointer.  Checks, all exact:
 *   - SpMV of the reference's known answer A = [1 0 2; 0 3 0; 4 0 5],
 *     x = [1, 2, 3] -> y = [7, 6, 19] (test/test_emitter.jl:97-135), 1-based
 *     and 0-based;
 *   - a prepared SpMV plan: create, execute with alpha and beta, new values,
 *     execute, destroy;
 *   - SpMM of the same A with B = [e1, 2 e2 + e3]: C = [A e1, 2 A e2 + A e3];
 *   - SDDMM over A's pattern with A = I and B = ones: every entry 1;
 *   - BSR SpMV (fp32, 2 x 2 blocks) of diag([1 2; 3 4], [5 6; 7 8]) times
 *     ones: [3, 7, 11, 15];
 *   - BSR SpMM (fp64, one 16 x 16 block V[r][s] = r + s) times B with columns
 *     1 and s: C[r] = [16 r + 120, 120 r + 1240];
 *   - the error path: origin 2 gives JLUST_STATUS_INDEX_ORIGIN and a message.
 *
 * jlust_c_harness_run(msg, len) returns 0 when every check holds, else the
 * number of the first failing check, with a description in msg.
 */
#include <stdio.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "jlust_hip.h"

#define CHECK(cond, id, ...)                          \
    do {                                              \
        if (!(cond)) {                                \
            snprintf(msg, len, __VA_ARGS__);          \
            rc = (id);                                \
            goto done;                                \
        }                                             \
    } while (0)

static void *to_dev(const void *h, size_t bytes)
{
    void *d = NULL;
    if (hipMalloc(&d, bytes ? bytes : 4) != hipSuccess) return NULL;
    if (bytes && hipMemcpy(d, h, bytes, hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipFree(d);
        return NULL;
    }
    return d;
}

static int from_dev(void *h, const void *d, size_t bytes)
{
    return hipMemcpy(h, d, bytes, hipMemcpyDeviceToHost) == hipSuccess ? 0 : -1;
}

int jlust_c_harness_run(char *msg, size_t len)
{
    int rc = 0;
    void *d[32] = {0};
    int nd = 0;
    jlust_spmv_plan_t plan = NULL;
    snprintf(msg, len, "ok");

    /* A = [1 0 2; 0 3 0; 4 0 5] in CSR, 1-based (JLUST's default). */
    const int32_t rp1[4] = {1, 3, 4, 6}, ci1[5] = {1, 3, 2, 1, 3};
    const int32_t rp0[4] = {0, 2, 3, 5}, ci0[5] = {0, 2, 1, 0, 2};
    const double val[5] = {1, 2, 3, 4, 5}, x[3] = {1, 2, 3};
    double y[3] = {-1, -1, -1};
    int32_t *drp1, *dci1, *drp0, *dci0;
    double *dval, *dx, *dy;
    d[nd++] = drp1 = (int32_t *)to_dev(rp1, sizeof rp1);
    d[nd++] = dci1 = (int32_t *)to_dev(ci1, sizeof ci1);
    d[nd++] = drp0 = (int32_t *)to_dev(rp0, sizeof rp0);
    d[nd++] = dci0 = (int32_t *)to_dev(ci0, sizeof ci0);
    d[nd++] = dval = (double *)to_dev(val, sizeof val);
    d[nd++] = dx = (double *)to_dev(x, sizeof x);
    d[nd++] = dy = (double *)to_dev(y, sizeof y);
    for (int i = 0; i < nd; ++i) CHECK(d[i] != NULL, 1, "device allocation %d failed", i);
    CHECK(jlust_hip_version() == JLUST_HIP_ABI_VERSION, 2, "ABI version %d, header %d", jlust_hip_version(),
          JLUST_HIP_ABI_VERSION);

    /* Plain SpMV, both origins, on the null (default) stream. */
    for (int origin = 1; origin >= 0; --origin) {
        int st = jlust_hip_csr_spmv_f64_i32(3, 3, 5, origin, origin ? drp1 : drp0, origin ? dci1 : dci0, dval, 1.0,
                                           dx, 0.0, dy, NULL);
        CHECK(st == JLUST_STATUS_SUCCESS, 3, "csr_spmv origin %d: status %d (%s)", origin, st,
              jlust_hip_last_error());
        CHECK(hipDeviceSynchronize() == hipSuccess && from_dev(y, dy, sizeof y) == 0, 4, "copy back failed");
        CHECK(y[0] == 7 && y[1] == 6 && y[2] == 19, 5, "csr_spmv origin %d: y = [%g, %g, %g], want [7, 6, 19]",
              origin, y[0], y[1], y[2]);
    }

    /* Prepared plan: create, execute (alpha 2, beta 1 on y = [7, 6, 19]),
     * new values (all doubled), execute again with beta 0, destroy. */
    {
        int st = jlust_hip_csr_spmv_plan_create(3, 3, 5, 1, 0, drp1, dci1, dval, NULL, &plan);
        CHECK(st == JLUST_STATUS_SUCCESS && plan, 6, "plan_create: status %d (%s)", st, jlust_hip_last_error());
        st = jlust_hip_csr_spmv_plan_execute_f64(plan, 2.0, dx, 1.0, dy, NULL);
        CHECK(st == JLUST_STATUS_SUCCESS, 7, "plan_execute: status %d (%s)", st, jlust_hip_last_error());
        CHECK(hipDeviceSynchronize() == hipSuccess && from_dev(y, dy, sizeof y) == 0, 4, "copy back failed");
        CHECK(y[0] == 21 && y[1] == 18 && y[2] == 57, 8, "plan: y = [%g, %g, %g], want [21, 18, 57]", y[0], y[1],
              y[2]);
        const double val2[5] = {2, 4, 6, 8, 10};
        CHECK(hipMemcpy(dval, val2, sizeof val2, hipMemcpyHostToDevice) == hipSuccess, 4, "copy failed");
        st = jlust_hip_csr_spmv_plan_update_values(plan, dval, NULL);
        CHECK(st == JLUST_STATUS_SUCCESS, 9, "plan_update_values: status %d (%s)", st, jlust_hip_last_error());
        st = jlust_hip_csr_spmv_plan_execute_f64(plan, 1.0, dx, 0.0, dy, NULL);
        CHECK(st == JLUST_STATUS_SUCCESS, 7, "plan_execute: status %d (%s)", st, jlust_hip_last_error());
        CHECK(hipDeviceSynchronize() == hipSuccess && from_dev(y, dy, sizeof y) == 0, 4, "copy back failed");
        CHECK(y[0] == 14 && y[1] == 12 && y[2] == 38, 10, "plan after update: y = [%g, %g, %g], want [14, 12, 38]",
              y[0], y[1], y[2]);
        st = jlust_hip_csr_spmv_plan_destroy(plan);
        plan = NULL;
        CHECK(st == JLUST_STATUS_SUCCESS, 11, "plan_destroy: status %d (%s)", st, jlust_hip_last_error());
        CHECK(hipMemcpy(dval, val, sizeof val, hipMemcpyHostToDevice) == hipSuccess, 4, "copy failed");
    }

    /* SpMM: B = [1 0; 0 2; 0 1] (3 x 2, column-major), C = A * B. */
    {
        const double B[6] = {1, 0, 0, 0, 2, 1};           /* columns [1,0,0], [0,2,1] */
        const double want[6] = {1, 0, 4, 2, 6, 5};        /* A*[1,0,0] = [1,0,4]; A*[0,2,1] = [2,6,5] */
        double C[6];
        double *dB = (double *)to_dev(B, sizeof B), *dC = (double *)to_dev(B, sizeof B);
        d[nd++] = dB;
        d[nd++] = dC;
        CHECK(dB && dC, 1, "device allocation failed");
        int st = jlust_hip_csr_spmm_f64_i32(3, 3, 2, 5, 1, drp1, dci1, dval, 1.0, dB, 3, 0.0, dC, 3, 0, NULL);
        CHECK(st == JLUST_STATUS_SUCCESS, 12, "csr_spmm: status %d (%s)", st, jlust_hip_last_error());
        CHECK(hipDeviceSynchronize() == hipSuccess && from_dev(C, dC, sizeof C) == 0, 4, "copy back failed");
        for (int i = 0; i < 6; ++i)
            CHECK(C[i] == want[i], 13, "csr_spmm: C[%d] = %g, want %g", i, C[i], want[i]);
    }

    /* SDDMM over A's pattern: Cval[p] = dot(Amat[i,:], Bmat[:,j]) with
     * Amat = I (3 x 3) and Bmat = all ones -> every stored entry is 1. */
    {
        const double I3[9] = {1, 0, 0, 0, 1, 0, 0, 0, 1}, ones[9] = {1, 1, 1, 1, 1, 1, 1, 1, 1};
        double cv[5] = {-1, -1, -1, -1, -1};
        double *dI = (double *)to_dev(I3, sizeof I3), *dO = (double *)to_dev(ones, sizeof ones),
               *dcv = (double *)to_dev(cv, sizeof cv);
        d[nd++] = dI;
        d[nd++] = dO;
        d[nd++] = dcv;
        CHECK(dI && dO && dcv, 1, "device allocation failed");
        int st = jlust_hip_csr_sddmm_f64_i32(3, 3, 3, 5, 1, drp1, dci1, 1.0, dI, 3, dO, 3, 0.0, dcv, NULL, NULL);
        CHECK(st == JLUST_STATUS_SUCCESS, 14, "csr_sddmm: status %d (%s)", st, jlust_hip_last_error());
        CHECK(hipDeviceSynchronize() == hipSuccess && from_dev(cv, dcv, sizeof cv) == 0, 4, "copy back failed");
        for (int i = 0; i < 5; ++i) CHECK(cv[i] == 1, 15, "csr_sddmm: Cval[%d] = %g, want 1", i, cv[i]);
    }

    /* BSR SpMV, fp32, two 2 x 2 blocks on the diagonal, row-major, 1-based. */
    {
        const int32_t bp[3] = {1, 2, 3}, bc[2] = {1, 2};
        const float bv[8] = {1, 2, 3, 4, 5, 6, 7, 8}, bx[4] = {1, 1, 1, 1};
        float by[4] = {-1, -1, -1, -1};
        int32_t *dbp = (int32_t *)to_dev(bp, sizeof bp), *dbc = (int32_t *)to_dev(bc, sizeof bc);
        float *dbv = (float *)to_dev(bv, sizeof bv), *dbx = (float *)to_dev(bx, sizeof bx),
              *dby = (float *)to_dev(by, sizeof by);
        d[nd++] = dbp;
        d[nd++] = dbc;
        d[nd++] = dbv;
        d[nd++] = dbx;
        d[nd++] = dby;
        CHECK(dbp && dbc && dbv && dbx && dby, 1, "device allocation failed");
        int st = jlust_hip_bsr_spmv_f32_i32(2, 2, 2, 2, 2, 1, dbp, dbc, dbv, 1, 1.0f, dbx, 0.0f, dby, NULL);
        CHECK(st == JLUST_STATUS_SUCCESS, 18, "bsr_spmv: status %d (%s)", st, jlust_hip_last_error());
        CHECK(hipDeviceSynchronize() == hipSuccess && from_dev(by, dby, sizeof by) == 0, 4, "copy back failed");
        CHECK(by[0] == 3 && by[1] == 7 && by[2] == 11 && by[3] == 15, 19,
              "bsr_spmv: y = [%g, %g, %g, %g], want [3, 7, 11, 15]", by[0], by[1], by[2], by[3]);
    }

    /* BSR SpMM, fp64 matrix cores: one 16 x 16 block V[r][s] = r + s,
     * B = [ones, (0..15)] (16 x 2, column-major). */
    {
        const int32_t bp[2] = {1, 2}, bc[1] = {1};
        double bv[256], bB[32], bC[32];
        for (int r = 0; r < 16; ++r)
            for (int c = 0; c < 16; ++c) bv[r * 16 + c] = r + c;
        for (int r = 0; r < 16; ++r) {
            bB[r] = 1;
            bB[16 + r] = r;
        }
        int32_t *dbp = (int32_t *)to_dev(bp, sizeof bp), *dbc = (int32_t *)to_dev(bc, sizeof bc);
        double *dbv = (double *)to_dev(bv, sizeof bv), *dbB = (double *)to_dev(bB, sizeof bB),
               *dbC = (double *)to_dev(bB, sizeof bB);
        d[nd++] = dbp;
        d[nd++] = dbc;
        d[nd++] = dbv;
        d[nd++] = dbB;
        d[nd++] = dbC;
        CHECK(dbp && dbc && dbv && dbB && dbC, 1, "device allocation failed");
        int st = jlust_hip_bsr_spmm_f64_i32(1, 1, 16, 1, 1, dbp, dbc, dbv, 1, 2, 1.0, dbB, 16, 0.0, dbC, 16, NULL);
        CHECK(st == JLUST_STATUS_SUCCESS, 20, "bsr_spmm_f64: status %d (%s)", st, jlust_hip_last_error());
        CHECK(hipDeviceSynchronize() == hipSuccess && from_dev(bC, dbC, sizeof bC) == 0, 4, "copy back failed");
        for (int r = 0; r < 16; ++r)
            CHECK(bC[r] == 16.0 * r + 120 && bC[16 + r] == 120.0 * r + 1240, 21,
                  "bsr_spmm_f64: C[%d] = [%g, %g], want [%g, %g]", r, bC[r], bC[16 + r], 16.0 * r + 120,
                  120.0 * r + 1240);
    }

    /* Error path: origin 2 is neither 0 nor 1. */
    {
        int st = jlust_hip_csr_spmv_f64_i32(3, 3, 5, 2, drp1, dci1, dval, 1.0, dx, 0.0, dy, NULL);
        CHECK(st == JLUST_STATUS_INDEX_ORIGIN, 16, "bad origin: status %d, want %d", st, JLUST_STATUS_INDEX_ORIGIN);
        CHECK(strlen(jlust_hip_last_error()) > 0, 17, "bad origin: empty error message");
    }

done:
    if (plan) (void)jlust_hip_csr_spmv_plan_destroy(plan);
    (void)hipDeviceSynchronize();
    for (int i = 0; i < nd; ++i)
        if (d[i]) (void)hipFree(d[i]);
    return rc;
}
