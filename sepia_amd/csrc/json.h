/* json.h -- a small JSON reader for the on-disk sidecars (resident
 * manifest, sepia-index). Internal to libsepia_hip.so. */
#ifndef SEPIA_JSON_H
#define SEPIA_JSON_H

#include <stddef.h>
#include <stdint.h>

typedef enum { SJ_NULL, SJ_BOOL, SJ_NUM, SJ_STR, SJ_ARR, SJ_OBJ } SjType;

typedef struct SjValue {
    SjType type;
    int b;                  /* SJ_BOOL */
    int is_int;             /* SJ_NUM written without fraction or exponent, within int64 */
    int64_t i;              /* SJ_NUM as an integer (valid when is_int) */
    double d;               /* SJ_NUM */
    char *s;                /* SJ_STR, NUL-terminated UTF-8 */
    size_t n;               /* SJ_ARR / SJ_OBJ element count */
    struct SjValue **items; /* SJ_ARR elements, SJ_OBJ values */
    char **keys;            /* SJ_OBJ keys, parallel to items */
} SjValue;

/* Parses text[0, len). NULL on malformed input, with a message in err. */
__attribute__((visibility("hidden"))) SjValue *sj_parse(const char *text, size_t len, char *err, size_t errlen);
/* The value of key in an object (the first one), NULL if absent or obj is not an object. */
__attribute__((visibility("hidden"))) const SjValue *sj_get(const SjValue *obj, const char *key);
__attribute__((visibility("hidden"))) void sj_free(SjValue *v);

#endif
