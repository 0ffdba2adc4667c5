/* kvd_table.c -- the section-6b dispatch table of the HIP backend
 * (include/sp/sp_l1.h:403-410 layout), its copy-on-write fork hook and its
 * batched multi-session decode hook.
 * Plain C so the table is an ordinary host object. */
#include "sp_hipkv.h"

const sp_kvdecode_dispatch_fn sp_hipkv_dispatch = {
    sp_hipkv_open, sp_hipkv_prefill, sp_hipkv_decode_step,
    sp_hipkv_rewind, sp_hipkv_position, sp_hipkv_close,
};

__attribute__((constructor)) static void sp_hipkv_register_fork(void) {
    spx_register_fork(&sp_hipkv_dispatch, sp_hipkv_fork);
    spx_register_batch(&sp_hipkv_dispatch, sp_hipkv_decode_batch);
}
