/* ork/context.h -- device context lifecycle and introspection (MI355X build).
 * Part of <ork_npu.h>; include that. Each prototype names the reference declaration it replaces. */
#ifndef ORK_CONTEXT_H
#define ORK_CONTEXT_H

/* reference include/ork/context.h:13. Returns "1.0.190+mi355x". */
const char  *ork_npu_version(void);
/* reference include/ork/context.h:37. The O4N1 blob version written/accepted (1). */
uint32_t     ork_pack_format_version(void);

/* reference include/ork/context.h:68. Opens GPU 0 (or $ORK_HIP_DEVICE) and owns it for the process:
 * one HIP stream, staging buffers. NULL if no HIP device is present. ORK_USE_ORKD is ignored (there
 * is no daemon: single-process ownership). */
ork_npu     *ork_npu_init(void);
/* reference include/ork/context.h:73. No device: packs and loads keep the int8 codes [K][N] on the host
 * (ork_w_codes), and runs of those weights compute the exact result on the CPU, as the reference's offline
 * branches do (int8 / int4 runs, grouped runs, the int8 chain, the int4 chain and stream); fp16 runs and
 * the int8 / fp16 streams fail with -1 there. soc_id: "gfx950", "mi355x" (or the reference's
 * "rk3588"/"rk3576", accepted for blob tooling). NULL on an unknown id. */
ork_npu     *ork_npu_init_offline(const char *soc_id);
/* reference include/ork/context.h:83. Frees every device buffer the context still owns, including the
 * device memory of weights released with ork_w_free. */
void         ork_npu_free(ork_npu *ctx);

/* reference include/ork/context.h:96 / :18. The GPU architecture, "gfx950". */
const char  *ork_npu_soc(const ork_npu *ctx);
const char  *ork_npu_soc_id(ork_npu *ctx);
/* reference include/ork/context.h:98. Compute units of the device (256 on MI355X). */
int          ork_npu_cores(const ork_npu *ctx);
/* reference include/ork/context.h:100. 1 on gfx950 (the validated target), else 0. */
int          ork_npu_validated(const ork_npu *ctx);
/* reference include/ork/context.h:108. Policy hint; n<=0 means all. Stored and reported only: the
 * planner sizes grids for the whole device. */
void         ork_npu_set_core_budget(ork_npu *ctx, int n);
/* reference include/ork/context.h:148. Count of unexpected HIP failures in this process. */
long         ork_io_failures(void);
/* reference include/ork/context.h:149. Failures a recovery path provokes on purpose (the reference's
 * permitted ioctl failures). This build provokes none: always 0. */
long         ork_io_expected_failures(void);

#endif
