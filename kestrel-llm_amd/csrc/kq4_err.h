/* kq4_err.h - error reporting shared by the library's C host files: records the message that
 * kq4_last_error() returns for the calling thread and returns code. Defined in kq4_api.hip. */
#ifndef KQ4_ERR_H
#define KQ4_ERR_H

#ifdef __cplusplus
extern "C" {
#endif

int kq4_fail(int code, const char *fmt, ...) __attribute__((visibility("hidden")));

#ifdef __cplusplus
}
#endif
#endif
