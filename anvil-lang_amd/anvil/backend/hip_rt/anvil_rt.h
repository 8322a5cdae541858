// anvil_rt.h — host run-time of the libraries anvil.backend.hip generates (and the scalar helpers
// their kernels share with the host, marked ANVIL_HD).
//
// Everything here reproduces a format or a rule of the Anvil language, so that a program prints,
// draws, shuffles, reads and stores exactly what the reference interpreter does (anvil/interp.py,
// the definition of the language's semantics): the counter-based random numbers, Python's integer
// division, the default number format and NumPy-style tensor printing, the data-file readers, the
// EINW checkpoint file, the scan of a stdin line for a number. Each format is stated where it is
// implemented. The code is organised around this backend's needs: random keys are computed once
// per stream so kernels only hash the index, printing goes through one growable text buffer that is
// written out in one call, data files are read whole into memory and then decoded (one table of
// element decoders for the NumPy kinds), and a checkpoint is validated by one parser before a
// single tensor changes.
//
// A run-time error ends the program: `anvil: <message>` on stderr, exit status 1.
#pragma once
#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#include <unistd.h>
#include <zlib.h>

#ifndef ANVIL_HD
#define ANVIL_HD
#endif

// ======================================================================================== numbers
// Random numbers (interp.py:55-71). A stream's key mixes its number, a salt (0 and 1 for the two
// uniforms of a normal draw, 7 for shuffles) and the program's seed:
//     key = stream * 0x85EBCA77 + salt * 0xC2B2AE3D + seed + 0x632BE5AB            (mod 2^32)
// element idx of the stream draws the 32 bits h(h(idx * 0x9E3779B1 + key)), where h is Chris
// Wellons' lowbias32 hash (x ^= x >> 16; x *= 0x7FEB352D; x ^= x >> 15; x *= 0x846CA68B; x ^= x >> 16).
// A uniform number keeps the top 24 bits: (bits >> 8) * 2^-24 in [0, 1), or ((bits >> 8) + 1) * 2^-24
// in (0, 1] when the draw must not be 0 (the logarithm of Box-Muller). Both are exact in float.
ANVIL_HD static inline uint32_t anvil_key(uint32_t stream, uint32_t salt, uint32_t seed) {
    return 0x632BE5ABu + seed + salt * 0xC2B2AE3Du + stream * 0x85EBCA77u;
}
ANVIL_HD static inline uint32_t anvil_lowbias(uint32_t v) {
    v = (v ^ (v >> 16)) * 0x7FEB352Du;
    v = (v ^ (v >> 15)) * 0x846CA68Bu;
    return v ^ (v >> 16);
}
ANVIL_HD static inline uint32_t anvil_draw(uint32_t key, uint32_t idx) {
    return anvil_lowbias(anvil_lowbias(idx * 0x9E3779B1u + key));
}
ANVIL_HD static inline float anvil_unit(uint32_t key, uint32_t idx, int open_low) {
    const uint32_t top = (anvil_draw(key, idx) >> 8) + (open_low ? 1u : 0u);     // at most 2^24: exact
    return (float)top * 5.9604644775390625e-08f;                                   // * 2^-24: exact
}
ANVIL_HD static inline float anvil_uniform(uint32_t idx, uint32_t stream, uint32_t salt, uint32_t seed, int open_low) {
    return anvil_unit(anvil_key(stream, salt, seed), idx, open_low);
}

// Integers follow Python: a // b rounds toward minus infinity and a % b takes the divisor's sign
// (a == (a // b) * b + a % b); a divisor of 0 counts as 1, and INT_MIN // -1 wraps to INT_MIN as
// NumPy's int32 does (ops.py division rules; interp.py evaluates them with NumPy).
ANVIL_HD static inline int anvil_floordiv(int a, int b) {
    if (b == 0) b = 1;
    if (b == -1) return (int)(0u - (uint32_t)a);
    const int q = a / b;                                  // toward zero; |q * b| <= |a|
    return (q * b != a && ((a < 0) != (b < 0))) ? q - 1 : q;
}
ANVIL_HD static inline int anvil_floormod(int a, int b) {
    if (b == 0) b = 1;
    if (b == -1) return 0;
    return (int)((uint32_t)a - (uint32_t)anvil_floordiv(a, b) * (uint32_t)b);
}
// NumPy's float remainder: a - floor(a / b) * b computed exactly as fmod, moved into the divisor's
// sign; a zero result carries the divisor's sign (np.mod(3, -1.5) is -0.0).
ANVIL_HD static inline float anvil_pymodf(float a, float b) {
    float r = fmodf(a, b);
    if (r == 0.0f) return b < 0.0f ? -0.0f : 0.0f;
    if ((r < 0.0f) != (b < 0.0f)) r += b;
    return r;
}
// max and min propagate nan (NumPy's maximum/minimum); the integer ones are plain.
ANVIL_HD static inline float anvil_maxf(float a, float b) { return (a != a) ? a : (b != b) ? b : (a < b ? b : a); }
ANVIL_HD static inline float anvil_minf(float a, float b) { return (a != a) ? a : (b != b) ? b : (b < a ? b : a); }
ANVIL_HD static inline int anvil_maxi(int a, int b) { return a < b ? b : a; }
ANVIL_HD static inline int anvil_mini(int a, int b) { return b < a ? b : a; }
// argmax / argmin as np.argmax / np.argmin pick (interp.py:478-481): a nan beats every number and
// the first nan wins; among numbers the strictly larger (smaller) value, a tie to the smaller index.
// Does element (v, i) replace the running pick (best, at)? The relation orders (value, index)
// pairs totally, so partial picks may meet in any order (lane loops, wavefront and LDS trees).
template <bool MAX> ANVIL_HD static inline bool anvil_arg_better(float v, int i, float best, int at) {
    const bool vn = v != v, bn = best != best;
    if (vn || bn) return vn && (!bn || i < at);
    return (MAX ? v > best : v < best) || (v == best && i < at);
}
template <bool MAX> ANVIL_HD static inline bool anvil_arg_better(int v, int i, int best, int at) {
    return (MAX ? v > best : v < best) || (v == best && i < at);
}
// Partial picks over consecutive chunks of a whole-tensor reduction (no output index), combined as
// the interpreter combines them (interp.py:484-516): a later chunk replaces the pick only if its
// extreme (np.max / np.min: nan when the chunk holds one) is strictly better, so a nan in the
// first chunk stays and a later chunk holding a nan is passed over.
template <bool MAX> ANVIL_HD static inline bool anvil_chunk_better(float part, float acc) {
    return MAX ? part > acc : part < acc;
}
template <bool MAX> ANVIL_HD static inline bool anvil_chunk_better(int part, int acc) {
    return MAX ? part > acc : part < acc;
}
// sign keeps 0, -0 and nan as they are (np.sign).
ANVIL_HD static inline float anvil_signf(float a) { return a > 0.0f ? 1.0f : (a < 0.0f ? -1.0f : a); }
ANVIL_HD static inline int anvil_signi(int a) { return (0 < a) - (a < 0); }
ANVIL_HD static inline float anvil_sigmoidf(float a) { return 1.0f / (1.0f + expf(-a)); }
// i32(x) truncates toward zero.
ANVIL_HD static inline int anvil_trunci(float a) { return (int)truncf(a); }
// i32 arithmetic wraps modulo 2^32.
ANVIL_HD static inline int anvil_wrap_add(int a, int b) { return (int)((uint32_t)a + (uint32_t)b); }
ANVIL_HD static inline int anvil_wrap_sub(int a, int b) { return (int)((uint32_t)a - (uint32_t)b); }
ANVIL_HD static inline int anvil_wrap_mul(int a, int b) { return (int)((uint32_t)a * (uint32_t)b); }

// ======================================================================================== host state
// The random state: `seed(n)` sets the seed and restarts the stream count; every kernel that draws
// takes the next stream, and so does every shuffle (interp.py:252-256, 309-320).
struct anvil_host_state {
    uint32_t seed;
    uint32_t stream;
    uint32_t seed0;     // the seed the library was generated with: library calls start from it
    double t0;          // clock() counts from here
};
static anvil_host_state anvil_hs = {0, 0, 0, 0.0};

static double anvil_seconds(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

[[noreturn]] static void anvil_die(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
static void anvil_die(const char *fmt, ...) {
    char msg[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(msg, sizeof msg, fmt, ap);
    va_end(ap);
    fflush(stdout);
    fprintf(stderr, "anvil: %s\n", msg);
    fflush(stderr);
    exit(1);
}

// A run-time check failed (an index out of range): what, and the value that broke it.
[[noreturn]] static void anvil_bad_value(const char *what, long long value) {
    anvil_die("runtime error: %s (got %lld)", what, value);
}

// ======================================================================================== text
// Everything a print statement writes is assembled in one buffer and handed to stdio in one call.
struct anvil_text { char *p; size_t len, cap; };

static void anvil_text_room(anvil_text *t, size_t more) {
    if (t->len + more + 1 <= t->cap) return;
    size_t cap = t->cap ? t->cap : 256;
    while (cap < t->len + more + 1) cap *= 2;
    char *p = (char *)realloc(t->p, cap);
    if (p == NULL) anvil_die("out of host memory (printing)");
    t->p = p;
    t->cap = cap;
}
static void anvil_text_put(anvil_text *t, const char *s, size_t n) {
    anvil_text_room(t, n);
    memcpy(t->p + t->len, s, n);
    t->len += n;
    t->p[t->len] = 0;
}
static void anvil_text_str(anvil_text *t, const char *s) { anvil_text_put(t, s, strlen(s)); }
static void anvil_text_fmt(anvil_text *t, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
static void anvil_text_fmt(anvil_text *t, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    char small[96];
    const int n = vsnprintf(small, sizeof small, fmt, ap);
    va_end(ap);
    if (n < 0) return;
    if ((size_t)n < sizeof small) { anvil_text_put(t, small, (size_t)n); return; }
    anvil_text_room(t, (size_t)n);
    va_start(ap, fmt);
    vsnprintf(t->p + t->len, (size_t)n + 1, fmt, ap);
    va_end(ap);
    t->len += (size_t)n;
}
static void anvil_text_write(anvil_text *t, FILE *f) {
    if (t->len) fwrite(t->p, 1, t->len, f);
    free(t->p);
    t->p = NULL;
    t->len = t->cap = 0;
}

// The default number format (interp.py:74-81): fixed with four decimals when the value is 0, nan,
// or 1e-4 <= |v| < 1e6; four-decimal scientific otherwise. Integers print in full.
static void anvil_text_f32(anvil_text *t, float v) {
    if (v != v) { anvil_text_put(t, "nan", 3); return; }      // any nan, whatever its sign bit
    const double d = (double)v, m = fabs(d);
    const int fixed = v == 0.0f || (m >= 1e-4 && m < 1e6);
    anvil_text_fmt(t, fixed ? "%.4f" : "%.4e", d);
}
// A value for a `{x:fmt}` item: Python formats every nan as "nan", printf a negative one as "-nan".
static inline double anvil_fmt_arg(float v) { return v != v ? (double)NAN : (double)v; }

// Tensors print as NumPy does (interp.py:84-115): nested brackets, elements of the last dimension
// separated by ", ", rows of dimension d by ",\n" and d + 1 spaces; "[]" when empty, the bare
// element at rank 0. Above 1000 elements every dimension longer than 6 shows its indices 0, 1, 2,
// "...", n-3, n-2, n-1 only.
#define ANVIL_ELLIPSIS (-1L)
struct anvil_tensor_view {
    const void *data;
    int is_int;
    int rank;
    const long *dims;
    long stride[16];
    long shown[16][7];      // the indices each dimension shows when summarized
    int count[16];          // how many (0: all of them)
};

static void anvil_text_elem(anvil_text *t, const anvil_tensor_view *v, long at) {
    if (v->is_int) anvil_text_fmt(t, "%d", ((const int *)v->data)[at]);
    else anvil_text_f32(t, ((const float *)v->data)[at]);
}

static void anvil_text_block(anvil_text *t, const anvil_tensor_view *v, int d, long base) {
    const int last = d == v->rank - 1;
    const long n = v->count[d] ? v->count[d] : v->dims[d];
    anvil_text_put(t, "[", 1);
    for (long k = 0; k < n; k++) {
        if (k) {
            if (last) anvil_text_put(t, ", ", 2);
            else {
                anvil_text_put(t, ",\n", 2);
                for (int s = 0; s <= d; s++) anvil_text_put(t, " ", 1);
            }
        }
        const long i = v->count[d] ? v->shown[d][k] : k;
        if (i == ANVIL_ELLIPSIS) anvil_text_put(t, "...", 3);
        else if (last) anvil_text_elem(t, v, base + i);
        else anvil_text_block(t, v, d + 1, base + i * v->stride[d]);
    }
    anvil_text_put(t, "]", 1);
}

static void anvil_text_tensor(anvil_text *t, const void *data, int is_int, int rank, const long *dims) {
    anvil_tensor_view v;
    v.data = data;
    v.is_int = is_int;
    v.rank = rank;
    v.dims = dims;
    if (rank == 0) { anvil_text_elem(t, &v, 0); return; }
    long numel = 1;
    for (int d = rank - 1; d >= 0; d--) { v.stride[d] = numel; numel *= dims[d]; }
    if (numel == 0) { anvil_text_put(t, "[]", 2); return; }
    for (int d = 0; d < rank; d++) {
        const long n = dims[d];
        v.count[d] = 0;
        if (numel > 1000 && n > 6) {
            const long pick[7] = {0, 1, 2, ANVIL_ELLIPSIS, n - 3, n - 2, n - 1};
            memcpy(v.shown[d], pick, sizeof pick);
            v.count[d] = 7;
        }
    }
    anvil_text_block(t, &v, 0, 0);
}

// `{k:...}` over a list of strings picks one ("?" out of range); chars() writes byte values as text;
// show() draws a grid of small integers with one glyph each ("?" out of range), a row per line.
static void anvil_text_pick(anvil_text *t, int k, const char *const *choices, int n) {
    anvil_text_str(t, (k >= 0 && k < n) ? choices[k] : "?");
}
static void anvil_text_chars(anvil_text *t, const int *codes, long n) {
    anvil_text_room(t, (size_t)n);
    for (long i = 0; i < n; i++) t->p[t->len + i] = (char)(codes[i] & 0xFF);
    t->len += (size_t)n;
    t->p[t->len] = 0;
}
static void anvil_show_grid(const int *grid, long rows, long cols, const char *const *glyphs, int n) {
    anvil_text t = {NULL, 0, 0};
    for (long at = 0; at < rows * cols; at++) {
        const int v = grid[at];
        anvil_text_str(&t, (v >= 0 && v < n) ? glyphs[v] : "?");
        if (at % cols == cols - 1) anvil_text_put(&t, "\n", 1);
    }
    anvil_text_write(&t, stdout);
}

// ======================================================================================== data files
// A data file is opened at the path the program was compiled with or, with $ANVIL_DATA set, under
// that directory by its file name (for a library built on one machine and run on another).
static const char *anvil_data_file(const char *path) {
    static char moved[4096];
    const char *dir = getenv("ANVIL_DATA");
    if (dir == NULL || *dir == 0) return path;
    const char *base = strrchr(path, '/');
    snprintf(moved, sizeof moved, "%s/%s", dir, base ? base + 1 : path);
    return moved;
}

// Files the program writes (save_npy, checkpoints) and the checkpoints it loads are at their
// compiled paths or, with $ANVIL_OUT set, in that directory under their file names: a run can keep
// its outputs apart without a new build (no counterpart in the reference, whose paths are fixed).
static const char *anvil_out_file(const char *path) {
    static char moved[4096];
    const char *dir = getenv("ANVIL_OUT");
    if (dir == NULL || *dir == 0) return path;
    const char *base = strrchr(path, '/');
    snprintf(moved, sizeof moved, "%s/%s", dir, base ? base + 1 : path);
    return moved;
}

[[noreturn]] static void anvil_wrong_shape(const char *path) {
    anvil_die("data file %s does not have the shape this program was compiled for", path);
}

// The whole file in memory (a NUL after its last byte); gunzip: through zlib, which reads a file
// that is not compressed as it is.
struct anvil_blob { unsigned char *p; long n; };

static anvil_blob anvil_blob_read(const char *path, int gunzip) {
    anvil_blob b = {NULL, 0};
    long cap = 1 << 16;
    b.p = (unsigned char *)malloc((size_t)cap + 1);
    if (b.p == NULL) anvil_die("out of host memory (reading %s)", path);
    if (gunzip) {
        gzFile z = gzopen(path, "rb");
        if (z == NULL) { free(b.p); anvil_die("cannot open data file %s", path); }
        for (;;) {
            if (b.n == cap) {
                cap *= 2;
                b.p = (unsigned char *)realloc(b.p, (size_t)cap + 1);
                if (b.p == NULL) anvil_die("out of host memory (reading %s)", path);
            }
            const int got = gzread(z, b.p + b.n, (unsigned)(cap - b.n));
            if (got <= 0) break;
            b.n += got;
        }
        gzclose(z);
    } else {
        FILE *f = fopen(path, "rb");
        if (f == NULL) { free(b.p); anvil_die("cannot open data file %s", path); }
        size_t got;
        while ((got = fread(b.p + b.n, 1, (size_t)(cap - b.n), f)) > 0) {
            b.n += (long)got;
            if (b.n == cap) {
                cap *= 2;
                b.p = (unsigned char *)realloc(b.p, (size_t)cap + 1);
                if (b.p == NULL) anvil_die("out of host memory (reading %s)", path);
            }
        }
        fclose(f);
    }
    b.p[b.n] = 0;
    return b;
}

// IDX (MNIST) files, gzip'ed or not: after `header` bytes, one unsigned byte per element.
static void anvil_read_idx(const char *path, void *out, long n, long header, int is_int) {
    path = anvil_data_file(path);
    anvil_blob b = anvil_blob_read(path, 1);
    if (b.n < header + n) { free(b.p); anvil_wrong_shape(path); }
    const unsigned char *px = b.p + header;
    for (long i = 0; i < n; i++) {
        if (is_int) ((int *)out)[i] = px[i];
        else ((float *)out)[i] = (float)px[i];
    }
    free(b.p);
}

// The numbers of a text file: every match of [-+]?(digits[.digits*]|.digits)([eE][-+]?digits)? in
// order (interp.py:28). Returns the length of the match at p, or 0 when none starts there.
static long anvil_number_at(const char *p) {
    const char *q = p;
    if (*q == '+' || *q == '-') q++;
    const char *d = q;
    while (*q >= '0' && *q <= '9') q++;
    const long whole = q - d;
    long frac = 0;
    if (*q == '.') {
        const char *f = ++q;
        while (*q >= '0' && *q <= '9') q++;
        frac = q - f;
        if (whole == 0 && frac == 0) return 0;
    } else if (whole == 0) {
        return 0;
    }
    if (*q == 'e' || *q == 'E') {
        const char *e = q + 1;
        if (*e == '+' || *e == '-') e++;
        const char *x = e;
        while (*e >= '0' && *e <= '9') e++;
        if (e > x) q = e;
    }
    return q - p;
}

// The text's number at p (len characters) as the nearest float.
static float anvil_number_value(const char *p, long len) {
    char tmp[128];
    if (len >= (long)sizeof tmp) len = sizeof tmp - 1;
    memcpy(tmp, p, (size_t)len);
    tmp[len] = 0;
    return strtof(tmp, NULL);
}

// CSV: skip `skip_lines` lines, then the first n numbers (anywhere: separators are not checked).
static void anvil_read_csv(const char *path, float *out, long n, long skip_lines) {
    path = anvil_data_file(path);
    anvil_blob b = anvil_blob_read(path, 0);
    const char *p = (const char *)b.p, *end = p + b.n;
    for (long s = 0; s < skip_lines && p < end; s++) {
        const char *nl = (const char *)memchr(p, '\n', (size_t)(end - p));
        p = nl ? nl + 1 : end;
    }
    long got = 0;
    while (got < n && p < end) {
        const long len = anvil_number_at(p);
        if (len == 0) { p++; continue; }
        out[got++] = anvil_number_value(p, len);
        p += len;
    }
    free(b.p);
    if (got < n) anvil_wrong_shape(path);
}

// A file's bytes, one element each: the file must hold exactly n.
static void anvil_read_bytes(const char *path, int *out, long n) {
    path = anvil_data_file(path);
    anvil_blob b = anvil_blob_read(path, 0);
    if (b.n != n) { free(b.p); anvil_wrong_shape(path); }
    for (long i = 0; i < n; i++) out[i] = b.p[i];
    free(b.p);
}

// NumPy element kinds (the code the front end records for a .npy or .safetensors tensor): 0 <f4,
// 1 <f8, 2 <f2, 3 <i4, 4 <i8, 5 u1, 6 i1, 7 <u2, 8 <i2; little-endian. The float kinds fill an f32
// tensor (f8 rounds to nearest), the integer kinds an i32 one (i8 keeps its low 32 bits).
static uint64_t anvil_le(const unsigned char *p, int bytes) {
    uint64_t v = 0;
    for (int i = bytes - 1; i >= 0; i--) v = (v << 8) | p[i];
    return v;
}
// IEEE half to float, exactly: the same value with an 8-bit exponent (subnormal halves normalised).
static float anvil_half(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu, bits;
    if (exp == 0x1F) bits = sign | 0x7F800000u | (man << 13);              // inf, nan
    else if (exp != 0) bits = sign | ((exp + 112u) << 23) | (man << 13);   // 127 - 15 = 112
    else if (man == 0) bits = sign;                                         // +-0
    else {                                                                  // subnormal: shift in
        int e = 113;
        while (!(man & 0x400u)) { man <<= 1; e--; }
        bits = sign | ((uint32_t)e << 23) | ((man & 0x3FFu) << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}
static double anvil_npy_f4(const unsigned char *p) { uint32_t u = (uint32_t)anvil_le(p, 4); float f; memcpy(&f, &u, 4); return f; }
static double anvil_npy_f8(const unsigned char *p) { uint64_t u = anvil_le(p, 8); double d; memcpy(&d, &u, 8); return d; }
static double anvil_npy_f2(const unsigned char *p) { return anvil_half((uint16_t)anvil_le(p, 2)); }
static int64_t anvil_npy_i4(const unsigned char *p) { return (int32_t)(uint32_t)anvil_le(p, 4); }
static int64_t anvil_npy_i8(const unsigned char *p) { return (int64_t)anvil_le(p, 8); }
static int64_t anvil_npy_u1(const unsigned char *p) { return p[0]; }
static int64_t anvil_npy_i1(const unsigned char *p) { return (int8_t)p[0]; }
static int64_t anvil_npy_u2(const unsigned char *p) { return (uint16_t)anvil_le(p, 2); }
static int64_t anvil_npy_i2(const unsigned char *p) { return (int16_t)(uint16_t)anvil_le(p, 2); }
struct anvil_npy_kind { int bytes; double (*real)(const unsigned char *); int64_t (*whole)(const unsigned char *); };
static const anvil_npy_kind anvil_npy_kinds[9] = {
    {4, anvil_npy_f4, NULL}, {8, anvil_npy_f8, NULL}, {2, anvil_npy_f2, NULL},
    {4, NULL, anvil_npy_i4}, {8, NULL, anvil_npy_i8}, {1, NULL, anvil_npy_u1},
    {1, NULL, anvil_npy_i1}, {2, NULL, anvil_npy_u2}, {2, NULL, anvil_npy_i2},
};

// n elements of `kind` from byte `offset`: a whole .npy must end right after them; kind + 16 marks a
// tensor inside a .safetensors file, which other tensors follow.
static void anvil_read_npy(const char *path, void *out, long n, long offset, int kind, int size) {
    path = anvil_data_file(path);
    const int slice = (kind & 16) != 0;
    kind &= 15;
    if (kind > 8 || anvil_npy_kinds[kind].bytes != size) anvil_wrong_shape(path);
    const anvil_npy_kind *k = &anvil_npy_kinds[kind];
    anvil_blob b = anvil_blob_read(path, 0);
    const long need = offset + n * (long)size;
    if (slice ? b.n < need : b.n != need) { free(b.p); anvil_wrong_shape(path); }
    const unsigned char *p = b.p + offset;
    for (long i = 0; i < n; i++, p += size) {
        if (k->real) ((float *)out)[i] = (float)k->real(p);
        else ((int *)out)[i] = (int)(uint32_t)(uint64_t)k->whole(p);
    }
    free(b.p);
}

// save_npy: the .npy header the front end built, then the raw 4-byte elements. A file that cannot
// be written is reported, and the program goes on.
static void anvil_write_npy(const char *path, const unsigned char *header, long hlen, const void *data, long bytes) {
    path = anvil_out_file(path);
    FILE *f = fopen(path, "wb");
    if (f == NULL) { fprintf(stderr, "anvil: cannot write %s\n", path); return; }
    fwrite(header, 1, (size_t)hlen, f);
    fwrite(data, 1, (size_t)bytes, f);
    fclose(f);
}

// ======================================================================================== checkpoints
// An EINW file (interp.py:341-372, ir.py:753-764), little-endian:
//     "EINW"  u32 version (2)  u64 tensor count n  |  n x u64 key  |  the tensors' 4-byte elements
// A key holds the tensor's element count in its low 32 bits and, in version 2, a 32-bit FNV-1a hash
// of "<name inside the model>:<dtype>:<d0,d1,...>" (never 0) in its high 32 bits; a version-1 file
// stores the counts alone. load() accepts version 1 or 2, the same n, equal keys (or counts) and
// exactly the bytes they imply; anything else (or no file) leaves every tensor as it was and
// gives 0, success gives 1.
struct anvil_ckpt_entry { void *data; uint64_t key; };

static uint64_t anvil_ckpt_elems(uint64_t key) { return key & 0xFFFFFFFFull; }

static void anvil_ckpt_save(const char *path, const anvil_ckpt_entry *tab, long n) {
    path = anvil_out_file(path);
    FILE *f = fopen(path, "wb");
    if (f == NULL) { fprintf(stderr, "anvil: cannot write %s\n", path); return; }
    unsigned char head[16] = {'E', 'I', 'N', 'W', 2, 0, 0, 0};
    for (int i = 0; i < 8; i++) head[8 + i] = (unsigned char)((uint64_t)n >> (8 * i));
    fwrite(head, 1, sizeof head, f);
    for (long t = 0; t < n; t++) {
        unsigned char k[8];
        for (int i = 0; i < 8; i++) k[i] = (unsigned char)(tab[t].key >> (8 * i));
        fwrite(k, 1, 8, f);
    }
    for (long t = 0; t < n; t++) fwrite(tab[t].data, 4, (size_t)anvil_ckpt_elems(tab[t].key), f);
    fclose(f);
}

// The byte offset of the first tensor if `file` is a checkpoint of exactly these tensors, else -1.
static long anvil_ckpt_parse(const unsigned char *file, long size, const anvil_ckpt_entry *tab, long n) {
    if (size < 16 || memcmp(file, "EINW", 4) != 0) return -1;
    const uint64_t version = anvil_le(file + 4, 4), count = anvil_le(file + 8, 8);
    if ((version != 1 && version != 2) || count != (uint64_t)n) return -1;
    const long data = 16 + 8 * n;
    if (size < data) return -1;
    uint64_t elems = 0;
    for (long t = 0; t < n; t++) {
        const uint64_t want = version == 2 ? tab[t].key : anvil_ckpt_elems(tab[t].key);
        if (anvil_le(file + 16 + 8 * t, 8) != want) return -1;
        elems += anvil_ckpt_elems(tab[t].key);
    }
    return (uint64_t)size == (uint64_t)data + 4 * elems ? data : -1;
}

static float anvil_ckpt_load(const char *path, const anvil_ckpt_entry *tab, long n) {
    path = anvil_out_file(path);
    FILE *f = fopen(path, "rb");
    if (f == NULL) return 0.0f;
    fclose(f);
    anvil_blob b = anvil_blob_read(path, 0);
    const long at = anvil_ckpt_parse(b.p, b.n, tab, n);
    if (at >= 0) {
        const unsigned char *p = b.p + at;
        for (long t = 0; t < n; t++) {
            const size_t bytes = 4 * (size_t)anvil_ckpt_elems(tab[t].key);
            memcpy(tab[t].data, p, bytes);
            p += bytes;
        }
    }
    free(b.p);
    return at >= 0 ? 1.0f : 0.0f;
}

// ======================================================================================== the rest
// Fisher-Yates from the back (interp.py:309-320): with the shuffle's own stream, the k-th step
// (k = 0 .. n-2) swaps p[i], i = n-1-k, with p[draw(k) mod (i + 1)].
static void anvil_fisher_yates(int *p, long n) {
    const uint32_t key = anvil_key(anvil_hs.stream++, 7u, anvil_hs.seed);
    for (long i = n - 1; i > 0; i--) {
        const long j = (long)(anvil_draw(key, (uint32_t)(n - 1 - i)) % (uint32_t)(i + 1));
        const int t = p[i];
        p[i] = p[j];
        p[j] = t;
    }
}

static void anvil_fill_iota(int *p, long n) {
    for (long i = 0; i < n; i++) p[i] = (int)i;
}

// nonzero: the first `size` flat indices of nonzero flags, in order, then -1 (interp.py:373-378).
static void anvil_find_nonzero(const int *flags, long n, int *out, long size) {
    long k = 0;
    for (long i = 0; i < n && k < size; i++)
        if (flags[i]) out[k++] = (int)i;
    if (k < size) {
        for (long r = k; r < size; r++) out[r] = -1;
    }
}

// input: one line of stdin; its first number (the grammar of anvil_number_at: decimal only, so
// "0x1F" reads 0) or nan when it has none (interp.py:332-340). At the end of the input: a newline,
// and 1 (the program ends).
static int anvil_read_number(float *out) {
    fflush(stdout);
    char *line = NULL;
    size_t cap = 0;
    const ssize_t len = getline(&line, &cap, stdin);
    if (len < 0) {
        free(line);
        fputs("\n", stdout);
        return 1;
    }
    float v = NAN;
    for (const char *p = line; *p; p++) {
        const long m = anvil_number_at(p);
        if (m > 0) { v = anvil_number_value(p, m); break; }
    }
    free(line);
    *out = v;
    return 0;
}
