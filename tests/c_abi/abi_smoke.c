/* Plain-C client of libtrntensor_hip.so: compiles against include/trntensor_hip.h
 * with a C compiler, links the library, and exercises the argument checks
 * that return before any device work (so it runs on a host without a GPU).
 * Exit status 0 when every check holds. */
#include <stdio.h>
#include <string.h>

#include "trntensor_hip.h"

static int fails = 0;

static void expect(int got, int want, const char* what) {
    if (got != want) {
        fprintf(stderr, "%s: status %d (%s), want %d: %s\n", what, got, tt_status_string(got), want, tt_last_error());
        ++fails;
    }
}

int main(void) {
    void* dummy = (void*)256;
    if (tt_abi_version() != TT_ABI_VERSION) {
        fprintf(stderr, "ABI version %d, header %d\n", tt_abi_version(), TT_ABI_VERSION);
        return 1;
    }
    /* empty GEMM: nothing to do */
    expect(tt_gemm(TT_F64, 0, 0, 0, 4, 4, 1.0, NULL, 4, 0, NULL, 4, 0, 0.0, NULL, 4, 0, NULL, 4, 0, 1, NULL), TT_OK,
           "empty gemm");
    expect(tt_gemm(TT_F64, 0, 0, -1, 4, 4, 1.0, NULL, 4, 0, NULL, 4, 0, 0.0, NULL, 4, 0, NULL, 4, 0, 1, NULL),
           TT_INVALID, "negative M");
    expect(tt_gemm(7, 0, 0, 4, 4, 4, 1.0, dummy, 4, 0, dummy, 4, 0, 0.0, NULL, 4, 0, dummy, 4, 0, 1, NULL),
           TT_UNSUPPORTED, "bad dtype");
    size_t ws = tt_mp2_energy_workspace_bytes(TT_F64, 64, 320, 1200);
    if (ws < (2080 * 15 + 1) * sizeof(double)) {
        fprintf(stderr, "mp2 workspace %zu too small\n", ws);
        ++fails;
    }
    expect(tt_mp2_energy(TT_F64, 64, 320, 1200, dummy, dummy, dummy, dummy, dummy, 8, 1, NULL), TT_INVALID,
           "mp2 small workspace");
    expect(tt_mp2_energy_noalloc(TT_F64, 2048, 1024, 64, dummy, dummy, dummy, dummy, 1, NULL), TT_INVALID,
           "mp2 noalloc beyond scratch");
    if (!strstr(tt_last_error(), "static scratch")) {
        fprintf(stderr, "noalloc message: %s\n", tt_last_error());
        ++fails;
    }
    int64_t shape[1] = {4};
    expect(tt_strided_contract(TT_I64, 1, shape, shape, shape, 0, shape, shape, shape, dummy, NULL, 0.5, 0.0, NULL, dummy,
                               NULL, 0, NULL),
           TT_INVALID, "int64 with a fractional alpha");
    expect(tt_hbm_probe(7, dummy, dummy, 64, 1, dummy, NULL), TT_INVALID, "hbm probe mode");
    expect(tt_hbm_probe(0, dummy, dummy, 24, 1, dummy, NULL), TT_INVALID, "hbm probe bytes not a multiple of 16");
    expect(tt_hbm_probe(0, NULL, dummy, 64, 1, dummy, NULL), TT_INVALID, "hbm probe read without src");
    if (fails == 0) printf("c abi ok\n");
    return fails ? 1 : 0;
}
