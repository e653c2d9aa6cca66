// Host check of neuroflow_amd/csrc/gelu_exact.h against glibc (the library
// the reference's tanhf comes from): tanhf_fdlibm on every float bit pattern
// with stride `stride` (1 = all 2^32), and gelu_ref against the reference
// expression 0.5f*z*(1 + tanhf(c*fma((0.044715f*z)*z, z, z))) with glibc
// (gelu_ref uses the straight-line tanhf_fdlibm_select, also compared)
// tanhf and c = sqrtf(2.0f / (float)M_PI).  Also the log2 snap's exponent
// (snap.h): the step table is located by scanning every float from 2^-6 to
// 2^10 with the reference's int(std::round(std::log2(a) * 8) / 8)
// (fno.cpp:579-606) under glibc, and snap_exponent_binade on that table is
// compared with the reference's exponent (capped at 9, where the snap
// saturates) on every float from 2^-6 to FLT_MAX with the same stride.
// Prints the mismatch counts.  Built with -ffp-contract=off.
#include <math.h>

#include <cmath>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>

#include "gelu_exact.h"
#include "snap.h"

static unsigned long long stride_g = 1;
static unsigned long long bad_tanh[16], bad_gelu[16], bad_sel[16], bad_snap[16];
static float thr_g[15];

static int snap_exponent_reference(float a) {
    const float r = std::round(std::log2(a) * 8.0f) / 8.0f;
    return static_cast<int>(r);
}
static const int kThreads = 8;

static float gelu_glibc(float z) {
    const float c = sqrtf(2.0f / (float)3.14159265358979323846);
    const float inner = fmaf((0.044715f * z) * z, z, z);
    return (0.5f * z) * (1.0f + tanhf(c * inner));
}

static void* run(void* arg) {
    const long id = (long)arg;
    unsigned long long bt = 0, bg = 0, bs = 0, bn = 0;
    for (unsigned long long u = (unsigned long long)id * stride_g; u < (1ull << 32); u += stride_g * kThreads) {
        const float x = nfq::gx_float((uint32_t)u);
        const float a = tanhf(x), b = nfq::tanhf_fdlibm(x);
        if (nfq::gx_bits(a) != nfq::gx_bits(b) && !(isnan(a) && isnan(b))) ++bt;
        const float c = nfq::tanhf_fdlibm_select(x);
        if (nfq::gx_bits(a) != nfq::gx_bits(c) && !(isnan(a) && isnan(c))) ++bs;
        const float ga = gelu_glibc(x), gb = nfq::gelu_ref(x);
        if (nfq::gx_bits(ga) != nfq::gx_bits(gb) && !(isnan(ga) && isnan(gb))) ++bg;
        if (u >= 0x3c800000u && u <= 0x7f7fffffu) {
            const int e = snap_exponent_reference(x);
            if (nfq::snap_exponent_binade(x, thr_g) != (e < 9 ? e : 9)) ++bn;
        }
    }
    bad_snap[id] = bn;
    bad_tanh[id] = bt;
    bad_gelu[id] = bg;
    bad_sel[id] = bs;
    return 0;
}

int main(int argc, char** argv) {
    stride_g = argc > 1 ? strtoull(argv[1], 0, 10) : 1;
    int steps = 0, e_prev = -6;   // the exponent at 2^-6
    for (uint32_t u = 0x3c800000u; u < 0x44800000u && steps < 15; ++u) {
        const int e = snap_exponent_reference(nfq::gx_float(u));
        for (; e_prev < e && steps < 15; ++e_prev) thr_g[steps++] = nfq::gx_float(u);
    }
    pthread_t th[kThreads];
    for (long i = 0; i < kThreads; ++i) pthread_create(&th[i], 0, run, (void*)i);
    unsigned long long bt = 0, bg = 0, bs = 0, bn = 0;
    for (int i = 0; i < kThreads; ++i) {
        pthread_join(th[i], 0);
        bt += bad_tanh[i];
        bg += bad_gelu[i];
        bs += bad_sel[i];
        bn += bad_snap[i];
    }
    const float c_ref = sqrtf(2.0f / (float)3.14159265358979323846);
    printf("tanh_mismatches %llu select_mismatches %llu gelu_mismatches %llu c_ok %d snap_steps %d "
           "snap_binned %d snap_mismatches %llu\n", bt, bs, bg, nfq::gx_bits(c_ref) == nfq::gx_bits(nfq::kGeluC),
           steps, (int)nfq::snap_table_binned(thr_g), bn);
    return 0;
}
