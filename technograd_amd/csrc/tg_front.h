/* The surface-language (.tg) front end: a model file, its imports and its
 * initializer files -> canonical TGIR text, the bytes the reference's
 * `tgc ir MODEL.tg` prints (src/parse.c, src/lower.c, src/ir.c:150-202).
 * Host code only; used by tg_hip_surface_to_tgir and `tgc-hip`. */
#ifndef TG_FRONT_H
#define TG_FRONT_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Lower the surface model at `path`. Returns malloc'd TGIR text, or NULL with
 * "file:line: message" (the reference's diagnostic) in err. */
char *tgf_lower(const char *path, char *err, size_t errn);

#ifdef __cplusplus
}
#endif

#endif
