/* Host-side checks of the C ABI (include/gdn_mi355x.h) under AddressSanitizer and UndefinedBehaviorSanitizer:
 * the size queries over many shapes and the argument checks that return before any device work (null pointers,
 * bad shapes, dtypes and forms, short buffers), the error strings, and the kernel-timing switch.  Built and run by
 * tests/test_abi_sanitize.py with the library's host code instrumented; needs no GPU.  Exits non-zero on the first
 * failed check. */
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "gdn_mi355x.h"

static int failures = 0;

#define CHECK(cond)                                                                 \
    do {                                                                            \
        if (!(cond)) {                                                              \
            fprintf(stderr, "check failed at line %d: %s\n", __LINE__, #cond);      \
            ++failures;                                                             \
        }                                                                           \
    } while (0)

static int err_has(const char *s) { return strstr(gdn_last_error(), s) != NULL; }

int main(void) {
    void *fake = (void *)(uintptr_t)256; /* never dereferenced: every call below fails its checks first */
    CHECK(gdn_version() > 0);

    /* forms */
    CHECK(gdn_select_form(32, 128, 128, 0, GDN_GATE_LOG, GDN_FORM_AUTO, GDN_F32) == GDN_FORM_CHUNK);
    CHECK(gdn_select_form(32, 128, 128, 1, GDN_GATE_LOG, GDN_FORM_AUTO, GDN_F32) == GDN_FORM_CHUNK);
    CHECK(gdn_select_form(32, 64, 128, 0, GDN_GATE_DECAY, GDN_FORM_AUTO, GDN_F32) == GDN_FORM_RECURRENT);
    CHECK(gdn_select_form(32, 128, 128, 0, GDN_GATE_DECAY_VEC, GDN_FORM_CHUNK, GDN_F32) == GDN_ERR_UNSUPPORTED);
    /* per-channel gates: the chunked form for bf16 inputs without a mask */
    CHECK(gdn_select_form(32, 128, 128, 0, GDN_GATE_DECAY_VEC, GDN_FORM_AUTO, GDN_BF16) == GDN_FORM_CHUNK);
    CHECK(gdn_select_form(32, 128, 128, 1, GDN_GATE_DECAY_VEC, GDN_FORM_AUTO, GDN_BF16) == GDN_FORM_RECURRENT);
    CHECK(gdn_saved_bytes(2, 300, 16, 32, 128, 128, 64, GDN_GATE_DECAY_VEC, 0, GDN_FORM_AUTO, GDN_BF16) >
          gdn_saved_bytes(2, 300, 16, 32, 128, 128, 64, GDN_GATE_LOG, 0, GDN_FORM_AUTO, GDN_BF16));
    CHECK(gdn_fwd_workspace_bytes(2, 300, 16, 32, 128, 128, 64, GDN_GATE_DECAY_VEC, 0, GDN_FORM_AUTO, GDN_BF16, 0) > 0);
    CHECK(gdn_bwd_workspace_bytes(2, 300, 16, 32, 128, 128, 256, GDN_GATE_DECAY_VEC, 0, GDN_FORM_AUTO, GDN_BF16) > 0);
    /* masked calls above 256 value heads: AUTO resolves to the recurrent form, and the size queries follow it */
    CHECK(gdn_select_form(260, 128, 128, 1, GDN_GATE_LOG, GDN_FORM_AUTO, GDN_F32) == GDN_FORM_RECURRENT);
    CHECK(gdn_select_form(260, 128, 128, 1, GDN_GATE_LOG, GDN_FORM_CHUNK, GDN_F32) == GDN_ERR_UNSUPPORTED && err_has("Hv <= 256"));
    CHECK(gdn_saved_bytes(1, 300, 130, 260, 128, 128, 64, GDN_GATE_LOG, 1, GDN_FORM_AUTO, GDN_BF16) ==
          gdn_saved_bytes(1, 300, 130, 260, 128, 128, 64, GDN_GATE_LOG, 1, GDN_FORM_RECURRENT, GDN_BF16));
    CHECK(gdn_bwd_workspace_bytes(1, 300, 130, 260, 128, 128, 64, GDN_GATE_LOG, 1, GDN_FORM_AUTO, GDN_BF16) ==
          gdn_bwd_workspace_bytes(1, 300, 130, 260, 128, 128, 64, GDN_GATE_LOG, 1, GDN_FORM_RECURRENT, GDN_BF16));
    CHECK(gdn_fwd_workspace_bytes(1, 300, 130, 260, 128, 128, 64, GDN_GATE_LOG, 1, GDN_FORM_AUTO, GDN_BF16, 1) == 0);
    {   /* a masked chunked call above 256 value heads is refused before anything runs */
        const int rc = gdn_fwd(fake, fake, fake, fake, fake, NULL, fake, fake, NULL, NULL, 0, NULL, 0, 1, 4, 130, 260,
                               128, 128, 64, GDN_BF16, GDN_BF16, GDN_GATE_LOG, GDN_FORM_CHUNK, NULL);
        CHECK(rc == GDN_ERR_UNSUPPORTED && err_has("Hv <= 256"));
    }

    /* size queries over shapes, dtypes, masks, chunks and forms */
    const int Ts[] = {1, 63, 64, 65, 200, 4096, 16384};
    const int chunks[] = {1, 16, 64, 100, 256};
    for (unsigned a = 0; a < sizeof Ts / sizeof Ts[0]; ++a)
        for (unsigned c = 0; c < sizeof chunks / sizeof chunks[0]; ++c)
            for (int mask = 0; mask < 2; ++mask)
                for (int dt = GDN_F32; dt <= GDN_BF16; ++dt)
                    for (int form = GDN_FORM_AUTO; form <= GDN_FORM_CHUNK; ++form) {
                        const int T = Ts[a], ch = chunks[c];
                        const size_t s = gdn_saved_bytes(2, T, 16, 32, 128, 128, ch, GDN_GATE_LOG, mask, form, dt);
                        const size_t wf = gdn_fwd_workspace_bytes(2, T, 16, 32, 128, 128, ch, GDN_GATE_LOG, mask,
                                                                  form, dt, 1);
                        const size_t wo = gdn_fwd_workspace_bytes(2, T, 16, 32, 128, 128, ch, GDN_GATE_LOG, mask,
                                                                  form, dt, 0);
                        const size_t wb = gdn_bwd_workspace_bytes(2, T, 16, 32, 128, 128, ch, GDN_GATE_LOG, mask,
                                                                  form, dt);
                        CHECK(wb > 0);
                        if (form == GDN_FORM_CHUNK) CHECK(wo > 0);
                        (void)s;
                        (void)wf;
                    }
    CHECK(gdn_saved_bytes(1, 4096, 16, 32, 128, 128, 64, GDN_GATE_LOG, 0, GDN_FORM_CHUNK, GDN_F32) >
          gdn_saved_bytes(1, 4096, 16, 32, 128, 128, 64, GDN_GATE_LOG, 0, GDN_FORM_RECURRENT, GDN_F32));
    /* checkpointing keeps ceil(T / W) - 1 snapshots */
    CHECK(gdn_saved_bytes(1, 2048, 16, 32, 128, 128, 256, GDN_GATE_DECAY, 0, GDN_FORM_CHUNK, GDN_F32) ==
          (size_t)7 * 32 * 128 * 128 * 4);
    CHECK(gdn_bwd_workspace_bytes(1, 4, 1, 1, 8, 8, 0, 0, 0, 0, 0) == 0);

    /* forward argument checks */
    int rc = gdn_fwd(NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, 0, NULL, 0, 1, 4, 2, 3, 8, 8, 0,
                     GDN_F32, GDN_F32, GDN_GATE_DECAY, GDN_FORM_AUTO, NULL);
    CHECK(rc == GDN_ERR_INVALID && err_has("chunk must be a positive integer"));
    rc = gdn_fwd(NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, 0, NULL, 0, 1, 4, 2, 3, 8, 8, 64,
                 GDN_F32, GDN_F32, GDN_GATE_DECAY, GDN_FORM_AUTO, NULL);
    CHECK(rc == GDN_ERR_INVALID && err_has("head count must divide"));
    rc = gdn_fwd(NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, 0, NULL, 0, 1, 4, 1, 1, 300, 8, 64,
                 GDN_F32, GDN_F32, GDN_GATE_DECAY, GDN_FORM_AUTO, NULL);
    CHECK(rc == GDN_ERR_UNSUPPORTED);
    rc = gdn_fwd(NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, 0, NULL, 0, 1, 4, 1, 1, 8, 8, 64, 7,
                 GDN_F32, GDN_GATE_DECAY, GDN_FORM_AUTO, NULL);
    CHECK(rc == GDN_ERR_INVALID && err_has("dtype"));
    rc = gdn_fwd(NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, 0, NULL, 0, 1, 4, 1, 1, 8, 8, 64,
                 GDN_F32, GDN_F32, GDN_GATE_DECAY, GDN_FORM_AUTO, NULL);
    CHECK(rc == GDN_ERR_INVALID && err_has("null"));
    rc = gdn_fwd(fake, fake, fake, fake, fake, fake, NULL, fake, fake, NULL, 0, NULL, 0, 1, 4, 1, 1, 128, 128, 64,
                 GDN_F32, GDN_F32, GDN_GATE_LOG, GDN_FORM_CHUNK, NULL);
    CHECK(rc == GDN_ERR_WORKSPACE && err_has("workspace of 0 bytes"));
    rc = gdn_fwd(fake, fake, fake, fake, fake, fake, NULL, fake, fake, fake, 16, NULL, 0, 1, 4, 1, 1, 128, 128, 64,
                 GDN_F32, GDN_F32, GDN_GATE_LOG, GDN_FORM_CHUNK, NULL);
    CHECK(rc == GDN_ERR_WORKSPACE && err_has("saved buffer of 16 bytes"));
    rc = gdn_fwd(fake, fake, fake, fake, fake, fake, (const uint8_t *)fake, fake, fake, fake, 16, NULL, 0, 1, 4, 1,
                 1, 128, 128, 64, GDN_F32, GDN_F32, GDN_GATE_LOG, GDN_FORM_CHUNK, NULL);
    CHECK(rc == GDN_ERR_WORKSPACE);
    CHECK(gdn_fwd(NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, 0, NULL, 0, 0, 4, 1, 1, 8, 8, 64,
                  GDN_F32, GDN_F32, GDN_GATE_DECAY, GDN_FORM_AUTO, NULL) == GDN_OK);

    /* backward argument checks */
    const size_t need = gdn_bwd_workspace_bytes(1, 4, 1, 1, 8, 8, 64, 0, 0, 0, 0);
    CHECK(need > 0);
    rc = gdn_bwd(fake, fake, fake, fake, fake, fake, fake, fake, 0, fake, fake, fake, fake, fake, fake, fake, fake,
                 fake, need - 1, 1, 4, 1, 1, 8, 8, 64, GDN_F32, GDN_F32, GDN_F32, GDN_GATE_DECAY, GDN_FORM_AUTO, NULL);
    CHECK(rc == GDN_ERR_WORKSPACE);
    rc = gdn_bwd(fake, fake, fake, fake, fake, fake, NULL, fake, (size_t)1 << 40, fake, fake, fake, fake, fake,
                 fake, fake, fake, fake, (size_t)1 << 40, 1, 4, 1, 1, 128, 128, 64, GDN_BF16, GDN_F16, GDN_BF16,
                 GDN_GATE_LOG, GDN_FORM_CHUNK, NULL);
    CHECK(rc == GDN_ERR_UNSUPPORTED && err_has("fp16"));

    /* the allocation-free forward and the decode step */
    rc = gdn_fwd_noalloc(fake, fake, fake, fake, fake, fake, (const uint8_t *)fake, fake, fake, 2, 70, 2, 4, 128, 128,
                         GDN_F32, GDN_F32, GDN_GATE_LOG, GDN_FORM_CHUNK, NULL);
    CHECK(rc == GDN_ERR_UNSUPPORTED && err_has("recurrent form only"));
    rc = gdn_fwd_noalloc(fake, fake, fake, fake, fake, fake, NULL, fake, fake, 16, 64, 16, 64, 128, 128, GDN_BF16,
                         GDN_BF16, GDN_GATE_LOG, GDN_FORM_CHUNK, NULL);
    CHECK(rc == GDN_ERR_UNSUPPORTED && err_has("fixed scratch"));
    CHECK(gdn_decode_step(fake, fake, fake, fake, fake, fake, fake, fake, 0, 1, 1, 8, 8, 0, 0, 0, NULL) == GDN_OK);
    CHECK(gdn_decode_step(fake, fake, fake, fake, fake, fake, fake, fake, 1, 1, 1, 300, 8, 0, 0, 0, NULL) ==
          GDN_ERR_UNSUPPORTED);
    CHECK(gdn_decode_step(fake, fake, fake, fake, fake, fake, fake, NULL, 1, 1, 1, 8, 8, 0, 0, 0, NULL) ==
          GDN_ERR_INVALID && err_has("null"));

    /* block ops */
    CHECK(gdn_gates_bwd_workspace_bytes(4096, 32) > 0);
    CHECK(gdn_conv_silu_bwd_workspace_bytes(2, 8192, 8192, 4) > 0);
    CHECK(gdn_gated_rmsnorm_bwd_workspace_bytes(4096, 128) > 0);
    CHECK(gdn_gates_fwd(NULL, NULL, NULL, NULL, NULL, NULL, 4, 300, GDN_F32, 0, 0, NULL) != GDN_OK);
    CHECK(gdn_l2norm_fwd(NULL, NULL, 4, 128, 1e-6f, 1.f, GDN_F32, NULL) != GDN_OK);

    /* the kernel-timing switch with nothing recorded */
    CHECK(gdn_profile_enable(1) == GDN_OK);
    char names[256];
    double ms[4];
    int counts[4];
    CHECK(gdn_profile_collect(4, names, 64, ms, counts) >= 0);
    CHECK(gdn_profile_enable(0) == GDN_OK);

    if (failures) {
        fprintf(stderr, "%d checks failed\n", failures);
        return 1;
    }
    printf("abi checks passed\n");
    return 0;
}
