/* jpeg.h -- this build's JPEG decoder (host/jpeg.c), used by the image
 * decoders of host/image.c; not part of the C-ABI headers. */
#ifndef AETCNN_JPEG_H
#define AETCNN_JPEG_H
#include <stddef.h>

/* A baseline / extended sequential JPEG in memory -> interleaved 8-bit
 * samples (*chans = 1 or 3, row-major, malloc'ed into *px).  0 on success;
 * -1 with *why set (a static message) on a malformed or unsupported file. */
int an_jpeg_decode(const unsigned char *buf, size_t len, int *W, int *H, int *chans,
                   unsigned char **px, const char **why);

#endif
