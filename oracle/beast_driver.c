/*
 * beast_driver.c — test infrastructure only (never linked into libspq4k).
 *
 * Exposes the reference's own beast_matvec (a static function of
 * desktop/beast_canyon/sp_beast_canyon.c:1122-1134, the BurnHard scalar
 * dequant-then-dot matvec) to the tests: this file includes that source file
 * where it lies under /root/reference and adds one exported wrapper. `make -C
 * oracle ref` compiles it with the flags the reference's CMake gives that file
 * under GCC (desktop/beast_canyon/CMakeLists.txt:52-54: -O3 -mfma -mf16c and
 * GCC's default fp contraction), with -march=native narrowed to x86-64-v3 so
 * the library loads on any AVX2 host (the loops it runs are element-wise or
 * serial, so the vector width does not change a result). Everything else in
 * the file is unreferenced and dropped by --gc-sections; the result links
 * with -z defs, against libc and libm only.
 */
#include "sp_beast_canyon.c"

__attribute__((visibility("default")))
int ref_beast_matvec(const void *W, unsigned type, const float *x, float *y, int n_out, int n_in) {
    float *scratch = (float *)malloc((size_t)n_in * sizeof(float));
    if (!scratch) return -1;
    sp_optane_tensor_t t;
    memset(&t, 0, sizeof t);
    t.ptr = (void *)W;
    t.type = type;
    beast_matvec(&t, x, y, scratch, n_out, n_in);
    free(scratch);
    return 0;
}
