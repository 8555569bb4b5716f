/* json.c -- recursive-descent JSON reader (RFC 8259) for the on-disk
 * sidecars: objects, arrays, strings with every escape (\uXXXX including
 * surrogate pairs, emitted as UTF-8), numbers (integers kept exactly in
 * int64 when written without a fraction or exponent), true/false/null.
 * Nesting is bounded (SJ_MAX_DEPTH) so hostile input cannot exhaust the
 * stack. */
#include "json.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define SJ_MAX_DEPTH 64

typedef struct {
    const char *p, *end;
    char *err;
    size_t errlen;
    int failed;
} SjCur;

static void sj_fail(SjCur *c, const char *what) {
    if (c->failed) return;
    c->failed = 1;
    if (c->err && c->errlen) snprintf(c->err, c->errlen, "%s", what);
}

static void sj_ws(SjCur *c) {
    while (c->p < c->end && (*c->p == ' ' || *c->p == '\t' || *c->p == '\n' || *c->p == '\r')) c->p++;
}

static SjValue *sj_new(SjType t) {
    SjValue *v = (SjValue *)calloc(1, sizeof(SjValue));
    if (v) v->type = t;
    return v;
}

void sj_free(SjValue *v) {
    if (!v) return;
    free(v->s);
    for (size_t i = 0; i < v->n; i++) {
        if (v->items) sj_free(v->items[i]);
        if (v->keys) free(v->keys[i]);
    }
    free(v->items);
    free(v->keys);
    free(v);
}

/* Growable byte buffer for strings. */
typedef struct {
    char *b;
    size_t n, cap;
} SjBuf;

static int sj_put(SjBuf *s, char ch) {
    if (s->n + 1 >= s->cap) {
        size_t cap = s->cap ? 2 * s->cap : 32;
        char *nb = (char *)realloc(s->b, cap);
        if (!nb) return 0;
        s->b = nb;
        s->cap = cap;
    }
    s->b[s->n++] = ch;
    return 1;
}

static int sj_put_utf8(SjBuf *s, uint32_t cp) {
    if (cp < 0x80) return sj_put(s, (char)cp);
    if (cp < 0x800) return sj_put(s, (char)(0xC0 | (cp >> 6))) && sj_put(s, (char)(0x80 | (cp & 0x3F)));
    if (cp < 0x10000)
        return sj_put(s, (char)(0xE0 | (cp >> 12))) && sj_put(s, (char)(0x80 | ((cp >> 6) & 0x3F))) &&
               sj_put(s, (char)(0x80 | (cp & 0x3F)));
    return sj_put(s, (char)(0xF0 | (cp >> 18))) && sj_put(s, (char)(0x80 | ((cp >> 12) & 0x3F))) &&
           sj_put(s, (char)(0x80 | ((cp >> 6) & 0x3F))) && sj_put(s, (char)(0x80 | (cp & 0x3F)));
}

static int sj_hex4(SjCur *c, uint32_t *out) {
    if (c->end - c->p < 4) return 0;
    uint32_t v = 0;
    for (int k = 0; k < 4; k++) {
        const char h = c->p[k];
        v <<= 4;
        if (h >= '0' && h <= '9') v |= (uint32_t)(h - '0');
        else if (h >= 'a' && h <= 'f') v |= (uint32_t)(h - 'a' + 10);
        else if (h >= 'A' && h <= 'F') v |= (uint32_t)(h - 'A' + 10);
        else return 0;
    }
    c->p += 4;
    *out = v;
    return 1;
}

/* c->p at the opening quote; returns the decoded string (malloc'd). */
static char *sj_string(SjCur *c) {
    SjBuf s = { NULL, 0, 0 };
    c->p++;
    for (;;) {
        if (c->p >= c->end) {
            sj_fail(c, "unterminated string");
            break;
        }
        const unsigned char ch = (unsigned char)*c->p++;
        if (ch == '"') {
            if (!sj_put(&s, '\0')) break;
            return s.b;
        }
        if (ch < 0x20) {
            sj_fail(c, "control character in string");
            break;
        }
        if (ch != '\\') {
            if (!sj_put(&s, (char)ch)) break;
            continue;
        }
        if (c->p >= c->end) {
            sj_fail(c, "unterminated escape");
            break;
        }
        const char e = *c->p++;
        int ok = 1;
        switch (e) {
        case '"': ok = sj_put(&s, '"'); break;
        case '\\': ok = sj_put(&s, '\\'); break;
        case '/': ok = sj_put(&s, '/'); break;
        case 'b': ok = sj_put(&s, '\b'); break;
        case 'f': ok = sj_put(&s, '\f'); break;
        case 'n': ok = sj_put(&s, '\n'); break;
        case 'r': ok = sj_put(&s, '\r'); break;
        case 't': ok = sj_put(&s, '\t'); break;
        case 'u': {
            uint32_t cp;
            if (!sj_hex4(c, &cp)) {
                sj_fail(c, "bad \\u escape");
                ok = 0;
                break;
            }
            if (cp >= 0xD800 && cp < 0xDC00) {
                uint32_t lo;
                if (c->end - c->p >= 2 && c->p[0] == '\\' && c->p[1] == 'u') {
                    c->p += 2;
                    if (!sj_hex4(c, &lo) || lo < 0xDC00 || lo >= 0xE000) {
                        sj_fail(c, "bad surrogate pair");
                        ok = 0;
                        break;
                    }
                    cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                } else {
                    sj_fail(c, "lone high surrogate");
                    ok = 0;
                    break;
                }
            } else if (cp >= 0xDC00 && cp < 0xE000) {
                sj_fail(c, "lone low surrogate");
                ok = 0;
                break;
            }
            ok = sj_put_utf8(&s, cp);
            break;
        }
        default:
            sj_fail(c, "unknown escape");
            ok = 0;
        }
        if (!ok) break;
    }
    sj_fail(c, "out of memory");
    free(s.b);
    return NULL;
}

static SjValue *sj_number(SjCur *c) {
    const char *start = c->p;
    int is_int = 1;
    if (c->p < c->end && *c->p == '-') c->p++;
    if (c->p >= c->end || *c->p < '0' || *c->p > '9') {
        sj_fail(c, "bad number");
        return NULL;
    }
    if (*c->p == '0') c->p++;
    else
        while (c->p < c->end && *c->p >= '0' && *c->p <= '9') c->p++;
    if (c->p < c->end && *c->p == '.') {
        is_int = 0;
        c->p++;
        if (c->p >= c->end || *c->p < '0' || *c->p > '9') {
            sj_fail(c, "bad fraction");
            return NULL;
        }
        while (c->p < c->end && *c->p >= '0' && *c->p <= '9') c->p++;
    }
    if (c->p < c->end && (*c->p == 'e' || *c->p == 'E')) {
        is_int = 0;
        c->p++;
        if (c->p < c->end && (*c->p == '+' || *c->p == '-')) c->p++;
        if (c->p >= c->end || *c->p < '0' || *c->p > '9') {
            sj_fail(c, "bad exponent");
            return NULL;
        }
        while (c->p < c->end && *c->p >= '0' && *c->p <= '9') c->p++;
    }
    const size_t len = (size_t)(c->p - start);
    char tmp[64];
    if (len >= sizeof tmp) {
        sj_fail(c, "number too long");
        return NULL;
    }
    memcpy(tmp, start, len);
    tmp[len] = '\0';
    SjValue *v = sj_new(SJ_NUM);
    if (!v) {
        sj_fail(c, "out of memory");
        return NULL;
    }
    v->d = strtod(tmp, NULL);
    if (is_int) {
        /* exact int64, or a double when it does not fit */
        int neg = tmp[0] == '-';
        uint64_t acc = 0;
        int over = 0;
        for (const char *q = tmp + neg; *q; q++) {
            const uint64_t dgt = (uint64_t)(*q - '0');
            if (acc > (UINT64_MAX - dgt) / 10) over = 1;
            acc = acc * 10 + dgt;
        }
        if (!over && acc <= (neg ? (uint64_t)INT64_MAX + 1 : (uint64_t)INT64_MAX)) {
            v->is_int = 1;
            v->i = neg ? (int64_t)(0 - acc) : (int64_t)acc;
        }
    }
    return v;
}

static int sj_lit(SjCur *c, const char *w) {
    const size_t n = strlen(w);
    if ((size_t)(c->end - c->p) < n || memcmp(c->p, w, n) != 0) return 0;
    c->p += n;
    return 1;
}

static SjValue *sj_value(SjCur *c, int depth);

static int sj_push(SjValue *v, SjValue *item, char *key, size_t *cap) {
    if (v->n == *cap) {
        const size_t ncap = *cap ? 2 * *cap : 8;
        SjValue **ni = (SjValue **)realloc(v->items, ncap * sizeof(SjValue *));
        if (!ni) return 0;
        v->items = ni;
        if (v->type == SJ_OBJ) {
            char **nk = (char **)realloc(v->keys, ncap * sizeof(char *));
            if (!nk) return 0;
            v->keys = nk;
        }
        *cap = ncap;
    }
    v->items[v->n] = item;
    if (v->type == SJ_OBJ) v->keys[v->n] = key;
    v->n++;
    return 1;
}

static SjValue *sj_container(SjCur *c, int depth, int obj) {
    SjValue *v = sj_new(obj ? SJ_OBJ : SJ_ARR);
    size_t cap = 0;
    if (!v) {
        sj_fail(c, "out of memory");
        return NULL;
    }
    c->p++;
    sj_ws(c);
    if (c->p < c->end && *c->p == (obj ? '}' : ']')) {
        c->p++;
        return v;
    }
    for (;;) {
        char *key = NULL;
        sj_ws(c);
        if (obj) {
            if (c->p >= c->end || *c->p != '"') {
                sj_fail(c, "expected a key");
                break;
            }
            key = sj_string(c);
            if (!key) break;
            sj_ws(c);
            if (c->p >= c->end || *c->p != ':') {
                free(key);
                sj_fail(c, "expected ':'");
                break;
            }
            c->p++;
        }
        SjValue *item = sj_value(c, depth + 1);
        if (!item || !sj_push(v, item, key, &cap)) {
            sj_free(item);
            free(key);
            sj_fail(c, "out of memory");
            break;
        }
        sj_ws(c);
        if (c->p < c->end && *c->p == ',') {
            c->p++;
            continue;
        }
        if (c->p < c->end && *c->p == (obj ? '}' : ']')) {
            c->p++;
            return v;
        }
        sj_fail(c, obj ? "expected ',' or '}'" : "expected ',' or ']'");
        break;
    }
    sj_free(v);
    return NULL;
}

static SjValue *sj_value(SjCur *c, int depth) {
    if (depth > SJ_MAX_DEPTH) {
        sj_fail(c, "nesting too deep");
        return NULL;
    }
    sj_ws(c);
    if (c->p >= c->end) {
        sj_fail(c, "unexpected end of input");
        return NULL;
    }
    const char ch = *c->p;
    if (ch == '{') return sj_container(c, depth, 1);
    if (ch == '[') return sj_container(c, depth, 0);
    if (ch == '"') {
        char *s = sj_string(c);
        if (!s) return NULL;
        SjValue *v = sj_new(SJ_STR);
        if (!v) {
            free(s);
            sj_fail(c, "out of memory");
            return NULL;
        }
        v->s = s;
        return v;
    }
    if (ch == '-' || (ch >= '0' && ch <= '9')) return sj_number(c);
    SjValue *v = NULL;
    if (sj_lit(c, "true")) {
        v = sj_new(SJ_BOOL);
        if (v) v->b = 1;
    } else if (sj_lit(c, "false")) {
        v = sj_new(SJ_BOOL);
    } else if (sj_lit(c, "null")) {
        v = sj_new(SJ_NULL);
    } else {
        sj_fail(c, "unexpected character");
        return NULL;
    }
    if (!v) sj_fail(c, "out of memory");
    return v;
}

SjValue *sj_parse(const char *text, size_t len, char *err, size_t errlen) {
    SjCur c = { text, text + len, err, errlen, 0 };
    if (err && errlen) err[0] = '\0';
    SjValue *v = sj_value(&c, 0);
    if (v) {
        sj_ws(&c);
        if (c.p != c.end) {
            sj_fail(&c, "trailing characters");
            sj_free(v);
            return NULL;
        }
    }
    if (!v && err && errlen && !err[0]) snprintf(err, errlen, "parse error");
    if (v && c.failed) {
        sj_free(v);
        return NULL;
    }
    return v;
}

const SjValue *sj_get(const SjValue *obj, const char *key) {
    if (!obj || obj->type != SJ_OBJ) return NULL;
    for (size_t i = 0; i < obj->n; i++)
        if (strcmp(obj->keys[i], key) == 0) return obj->items[i];
    return NULL;
}
