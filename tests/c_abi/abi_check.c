/* Plain C99 client of include/ullm_hip.h: compiles against the header alone
 * (no C++), links libullm_hip.so and exercises the host-side paths that need
 * no GPU -- version, workspace sizing, the RoPE table and the argument
 * validation / error codes of the attention entry points (all of which
 * return before any device work).  Exit status 0 = every check passed. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "ullm_hip.h"

static int failures = 0;
#define CHECK(cond)                                                    \
    do {                                                               \
        if (!(cond)) {                                                 \
            fprintf(stderr, "FAIL %s:%d: %s\n", __FILE__, __LINE__, #cond); \
            failures++;                                                \
        }                                                              \
    } while (0)

int main(void) {
    /* a fake, 16-byte aligned device address: never dereferenced, every call
       below fails validation first */
    void *fake = (void *)(uintptr_t)0x10000;
    const float *fq = (const float *)fake;
    float *fo = (float *)fake;
    const int32_t *fl = (const int32_t *)fake;

    CHECK(strncmp(ullm_hip_version(), "ullm-hip ", 9) == 0);

    /* workspace sizing: zero for a context one workgroup covers, positive
       for a split one, zero for bad shapes */
    CHECK(ullm_hip_decode_workspace_bytes(1, 12, 2, 128, 4096, 0) > 0);
    CHECK(ullm_hip_decode_workspace_bytes(1, 12, 5, 128, 4096, 0) == 0);
    CHECK(ullm_hip_decode_workspace_bytes(1, 12, 2, 96, 4096, 0) == 0);
    CHECK(ullm_hip_qkv_proj_workspace_bytes(1, 32, 8, 128) > 0);
    CHECK(ullm_hip_decode_noalloc_max_bytes() == (size_t)4 << 20);

    /* decode: each bad argument gets its documented code */
    CHECK(ullm_hip_attn_decode(fq, fake, fake, 7, 256, 0, fl, 100, 0, 1, 12, 2, 128, 0.1f, fo,
                               NULL, 0, NULL) == ULLM_HIP_E_UNSUPPORTED);
    CHECK(ullm_hip_attn_decode(fq, fake, fake, ULLM_DT_F16, 256, 0, fl, 100, 0, 1, 12, 2, 96,
                               0.1f, fo, NULL, 0, NULL) == ULLM_HIP_E_UNSUPPORTED);
    CHECK(ullm_hip_attn_decode(fq, fake, fake, ULLM_DT_F16, 256, 0, fl, 100, 0, 1, 12, 5, 128,
                               0.1f, fo, NULL, 0, NULL) == ULLM_HIP_E_INVALID);
    CHECK(ullm_hip_attn_decode(fq, fake, fake, ULLM_DT_F16, 100, 0, fl, 100, 0, 1, 12, 2, 128,
                               0.1f, fo, NULL, 0, NULL) == ULLM_HIP_E_INVALID);
    CHECK(ullm_hip_attn_decode(NULL, fake, fake, ULLM_DT_F16, 256, 0, fl, 100, 0, 1, 12, 2, 128,
                               0.1f, fo, NULL, 0, NULL) == ULLM_HIP_E_INVALID);
    CHECK(strstr(ullm_hip_last_error(), "null") != NULL);
    /* a split context without a workspace: E_WORKSPACE naming the size */
    CHECK(ullm_hip_attn_decode(fq, fake, fake, ULLM_DT_F16, 256, 0, fl, 4096, 0, 1, 12, 2, 128,
                               0.1f, fo, NULL, 0, NULL) == ULLM_HIP_E_WORKSPACE);
    CHECK(strstr(ullm_hip_last_error(), "bytes needed") != NULL);
    CHECK(ullm_hip_attn_decode_noalloc(fq, fake, fake, ULLM_DT_BF16, 256, 0, fl, 32768, 0, 1,
                                       16, 1, 256, 0.1f, fo, NULL) == ULLM_HIP_E_WORKSPACE);

    /* prefill: head_dim 96 is unsupported (any dtype), bad heads invalid */
    CHECK(ullm_hip_attn_prefill(fake, fake, fake, ULLM_DT_F32, 512, 16, 0, 0, 8, 2, 96, 0.1f, fo,
                                NULL) == ULLM_HIP_E_UNSUPPORTED);
    CHECK(ullm_hip_attn_prefill(fake, fake, fake, ULLM_DT_BF16, 256, 16, 0, 0, 8, 3, 128, 0.1f, fo,
                                NULL) != ULLM_HIP_OK);

    /* matmul: unsupported weight dtype */
    CHECK(ullm_hip_matmul(fake, ULLM_DT_F32, fq, fo, 256, 256, 16, NULL) == ULLM_HIP_E_UNSUPPORTED);

    /* the RoPE table (host): position 0 is (cos, sin) = (1, 0), bad sizes fail */
    {
        float cs[4 * 8 * 2];
        CHECK(ullm_hip_rope_table(cs, 4, 16, 10000.0f) == ULLM_HIP_OK);
        for (int i = 0; i < 8; i++) CHECK(cs[2 * i] == 1.0f && cs[2 * i + 1] == 0.0f);
        /* position 1, pair 0: angle 1 rad */
        CHECK(fabsf(cs[16] - cosf(1.0f)) < 1e-6f && fabsf(cs[17] - sinf(1.0f)) < 1e-6f);
        CHECK(ullm_hip_rope_table(cs, 4, 15, 10000.0f) == ULLM_HIP_E_INVALID);
        CHECK(ullm_hip_rope_table(NULL, 4, 16, 10000.0f) == ULLM_HIP_E_INVALID);
    }

    if (failures) {
        fprintf(stderr, "%d check(s) failed\n", failures);
        return 1;
    }
    printf("abi_check: all checks passed\n");
    return 0;
}
