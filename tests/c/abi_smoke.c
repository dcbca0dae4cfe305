/* Plain-C consumer of include/yoco_z1.h: compiled with gcc -std=c11 and linked against libyoco_z1.so by
 * tests/test_abi_host.py.  Without a GPU it only exercises calls that return before any device work. */
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "yoco_z1.h"

int main(void) {
    z1_table* t = 0;
    int bad = 0;
    bad |= z1_table_create(0, -1, Z1_F32, &t) != Z1_E_SIZE;
    bad |= z1_table_create(0, 0, 7, &t) != Z1_E_DTYPE;
    {   /* element counts beyond the grid's chunk limit are refused before any device call */
        float x[4];
        z1_tensor r[2];
        memset(r, 0, sizeof(r));
        r[0].g = x;
        r[0].n = INT64_MAX;
        bad |= z1_table_create(r, 1, Z1_F32, &t) != Z1_E_SIZE;
        r[0].n = (int64_t)INT32_MAX * 256 + 1;
        bad |= z1_table_create(r, 1, Z1_F32, &t) != Z1_E_SIZE;
        r[0].n = (int64_t)INT32_MAX * 128;       /* two rows whose chunks together exceed the limit */
        r[1] = r[0];
        bad |= z1_table_create(r, 2, Z1_F32, &t) != Z1_E_SIZE;
        bad |= t != 0;
    }
    bad |= z1_owner_sum_workspace(513) != Z1_NORM_PARTIALS + 3;       /* the partials, then one per 256-element chunk */
    bad |= z1_grad_norm_clip(0, 0, 0, 1.f, 0, 0, 0, 1.f, 0) != Z1_E_NULL;
    bad |= z1_table_set_grads(0, 0, 0, 0) != Z1_E_NULL;
    bad |= z1_adam_cast(0, 0, 0.f, 0.f, 0.f, 0.f, 1.f, 1.f, 0.f, 1, 0) != Z1_E_NULL;
    bad |= strlen(z1_strerror(Z1_E_WORKSPACE)) == 0;
    z1_update_scalars u;
    memset(&u, 0, sizeof(u));
    bad |= z1_update_scalars_run(0, &u, 0) != Z1_E_NULL;
    bad |= z1_grad_update_scalars(0, 0, &u, 0) != Z1_E_NULL;
    bad |= z1_embedding_backward_workspace(-1, 8, 10) != Z1_E_SIZE;
    bad |= z1_embedding_backward_workspace(16, 0, 10) != Z1_E_SIZE;
    bad |= z1_embedding_backward_workspace(16, (1 << 24) + 1, 10) != Z1_E_SIZE;
    bad |= z1_embedding_backward_workspace(16, 8, 10) <= 0;
    bad |= z1_adam_cast_dev(0, 0, 0.f, 0.f, 0.f, 0.f, 0, 0.f, 1, 0) != Z1_E_NULL;
    bad |= z1_adam_cast_rows(0, 0, 1, 0, 0.f, 0.f, 0.f, 0.f, 1.f, 1.f, 0.f, 1, 0) != Z1_E_NULL;
    bad |= z1_bias_corrections_step(0, 0.9, 0.95, 1, 0, 0) != Z1_E_NULL;
    printf("%s\n", bad ? "FAIL" : "ok");
    return bad;
}
