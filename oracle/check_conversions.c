/* Exhaustive conversion checker -- TEST INFRASTRUCTURE ONLY.
 *
 * usage: check_conversions <lib_a> <f32_to_f16_a> <f16_to_f32_a>
 *                          <lib_b> <f32_to_f16_b> <f16_to_f32_b> [stride]
 * Compares the two libraries' scalar conversions on every f16 bit pattern and
 * on every stride-th f32 bit pattern (stride 1 = all 2^32), bit for bit.
 * Prints the mismatch counts; exits 1 if any differ.
 */
#include <dlfcn.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef uint16_t (*narrow_fn)(float);
typedef float (*widen_fn)(uint16_t);

static void *sym(void *lib, const char *name) {
    void *p = dlsym(lib, name);
    if (p == NULL) {
        fprintf(stderr, "missing symbol %s\n", name);
        exit(2);
    }
    return p;
}

int main(int argc, char **argv) {
    if (argc < 7) {
        fprintf(stderr, "usage: %s lib_a narrow_a widen_a lib_b narrow_b widen_b [stride]\n", argv[0]);
        return 2;
    }
    void *a = dlopen(argv[1], RTLD_NOW | RTLD_LOCAL), *b = dlopen(argv[4], RTLD_NOW | RTLD_LOCAL);
    if (a == NULL || b == NULL) {
        fprintf(stderr, "dlopen failed: %s\n", dlerror());
        return 2;
    }
    narrow_fn na = (narrow_fn)sym(a, argv[2]), nb = (narrow_fn)sym(b, argv[5]);
    widen_fn wa = (widen_fn)sym(a, argv[3]), wb = (widen_fn)sym(b, argv[6]);
    const uint64_t stride = argc > 7 ? strtoull(argv[7], NULL, 10) : 1;
    unsigned long widen_bad = 0, narrow_bad = 0, checked = 0;
    for (uint32_t h = 0; h < 65536; h++) {
        const float x = wa((uint16_t)h), y = wb((uint16_t)h);
        if (memcmp(&x, &y, sizeof x) != 0) widen_bad++;
    }
    for (uint64_t u = 0; u < (1ull << 32); u += stride) {
        float f;
        const uint32_t bits = (uint32_t)u;
        memcpy(&f, &bits, sizeof f);
        if (na(f) != nb(f)) narrow_bad++;
        checked++;
    }
    printf("f16->f32 mismatches %lu of 65536; f32->f16 mismatches %lu of %lu\n", widen_bad,
           narrow_bad, checked);
    return widen_bad || narrow_bad ? 1 : 0;
}
