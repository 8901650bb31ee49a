/* A plain C99 caller of the C ABI (what a cgo, JNI or other C binding
 * compiles against): include/cast_amd.h must be valid C, and the host-only
 * entry points must answer without a GPU.  Prints one line per check and
 * exits non-zero on the first mismatch. */
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "cast_amd.h"

static int fail(const char *what) {
    printf("FAIL %s\n", what);
    return 1;
}

int main(void) {
    if (cast_abi_version() <= 0) return fail("abi version");
    printf("abi %d\n", cast_abi_version());
    if (strcmp(cast_status_string(CAST_OK), cast_status_string(CAST_ERR_SHAPE)) == 0) return fail("status strings");
    /* the headline shapes: 8 x (8192 + 128), 32/8 heads, D=128, bf16 */
    const size_t ws = cast_tree_attn_workspace_size(8, 1024, 66560, 32, 8, 128, CAST_BF16, 0);
    const int32_t split = cast_tree_attn_default_split(8, 1024, 66560, 32, 8, 128, CAST_BF16);
    printf("workspace %zu split %d\n", ws, (int)split);
    if (ws == 0 || split <= 0 || split % 64) return fail("split-K sizing");
    if (cast_tree_attn_workspace_size(8, 1024, 66560, 32, 8, 128, CAST_BF16, -1) != 0) return fail("no split");
    if (cast_tree_attn_noalloc_limit() < ws) return fail("no-allocation scratch below the headline's need");
    /* argument checks refuse before touching a device */
    if (cast_tree_bitmask(NULL, NULL, 1, 1, 2, NULL, NULL, NULL) != CAST_ERR_NULL_POINTER) return fail("null pointers");
    printf("ok\n");
    return 0;
}
