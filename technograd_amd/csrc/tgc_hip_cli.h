/* Shared pieces of the tgc-hip driver (tgc_hip_main.c) used by its stream and
 * serve commands (tgc_hip_serve.c). */
#ifndef TGC_HIP_CLI_H
#define TGC_HIP_CLI_H

#include <stddef.h>
#include <stdint.h>

/* numbers of one text row (f32, or Q16.16 words with `fixed`): the count, or -1 with *bad at the bad token */
int parse_row(const char *s, float *v, int max, const char **bad, int fixed);
/* a Q16.16 word with 6 decimals, as tg_fx_format prints it */
void fx_format(int32_t v, char *buf);
/* a model file's TGIR (the file, or a .tg model lowered); NULL with the reason in err */
char *load_model(const char *path, size_t *len, char *err, size_t errn);
/* SIGINT/SIGTERM set the stop signal; SIGPIPE ignored */
void install_signals(void);
int stop_signal(void);
int die(const char *fmt, const char *a);

int stream_main(int argc, char **argv);
int serve_main(int argc, char **argv);

#endif
