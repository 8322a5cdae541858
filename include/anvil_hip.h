/* anvil_hip.h — the C ABI of every library that anvil.backend.hip generates.
 *
 * A generated library is one Anvil program (or one function lowered by pyapi.lower) compiled for
 * MI355X (gfx950). It owns its device memory (one arena), its HIP stream and its host state; it is
 * not reentrant: callers serialize calls (the Python wrappers hold a lock, as the reference's
 * pyapi.Compiled does, pyapi.py:276, 286). A run-time error of the program (an index out of range,
 * a failed assert, a missing data file, a HIP error) prints `anvil: ...` on stderr and ends the
 * process with status 1, as the reference's compiled programs do (anvil_host.h:69-73;
 * anvil_cuda.h:91-103; pyapi.py:25-26).
 */
#ifndef ANVIL_HIP_ABI_H
#define ANVIL_HIP_ABI_H

#ifdef __cplusplus
extern "C" {
#endif

/* ---- running --------------------------------------------------------------------------------- */

/* Run the whole program from a fresh state (zeroed memory, constants loaded, the generated seed);
 * returns its exit status. Replaces the generated `int main(void)` of the reference's CUDA backend
 * (cuda.py:415-427), which `anvil run --cuda` executes as a process (cli.py:305-320). */
int anvil_main(void);

/* Library mode: one call of the lowered function. Inputs are read from the host arrays the
 * anvil_input<k> slots point to, results written to the host arrays of the anvil_output<k> slots.
 * The first call sets the library up; every call starts the random streams from the seed again.
 * Replaces the AArch64 library's `anvil_entry` (aarch64.py:141-142, 319-330, 357) that
 * pyapi.Compiled.call invokes (pyapi.py:282-299). */
int anvil_entry(void);

/* The same call with device pointers: the anvil_dinput<k> / anvil_doutput<k> slots hold device
 * addresses (a ROCm torch tensor's data_ptr()); the program reads and writes them in place, with
 * no host copies. It first waits for all device work. No counterpart in the reference (whose
 * ABI assumes host memory, pyapi.py:287-292): for callers whose data is already on the GPU. */
int anvil_entry_device(void);

/* One call of the lowered function that allocates nothing: no hipMalloc or hipFree, no pinned host
 * memory, no events or graphs. No counterpart in the reference; it is for callers that cannot
 * allocate (tight serving loops, harnesses that forbid it). It waits for `stream` before it
 * returns, so it cannot itself be recorded while that stream is being captured into a graph.
 * inputs[k] / outputs[k] are the device buffers of argument k and result k (input_bytes[k] /
 * output_bytes[k] must equal their compiled sizes: shapes are fixed when a function is lowered);
 * the work is queued on `stream` (a hipStream_t; NULL: the null stream) and the call returns after
 * it finished. The function's other buffers live in the library's static device array
 * `anvil_scratch`, one per GPU the library runs on, held until the process ends, at most
 * ANVIL_SCRATCH_MAX = 64 MiB and cleared at the start of every call. Calls that overlap on one GPU
 * share that array and race: serialize them. Returns 0, or, with a message on stderr and nothing
 * run: -1 wrong number of arguments, -2 an argument of the wrong size, -3 the function needs more
 * scratch than the maximum, -4 the library cannot run without allocating (it prints, reads data
 * files, checkpoints or was built with --check), -5 the scratch array is not found on the current
 * device. A run-time error of the program ends the process with status 1, as in anvil_entry. */
int anvil_entry_noalloc(void *const *inputs, const long long *input_bytes, int n_inputs,
                        void *const *outputs, const long long *output_bytes, int n_outputs, void *stream);

/* Set the library up (device, arena, constants) without running anything. */
int anvil_init(void);

/* Wait for the library's stream; reports (and exits on) a latched kernel fault. */
int anvil_sync_device(void);

/* ---- argument slots (library mode) ---------------------------------------------------------- */
/* For each argument k and result k of the lowered function, the library defines
 *     void *anvil_input<k>, *anvil_output<k>;     host pointers, set before anvil_entry()
 *     void *anvil_dinput<k>, *anvil_doutput<k>;   device pointers, set before anvil_entry_device()
 * (names of the reference's slots: aarch64.py:162-167, 945-949; pyapi.py:270-275). They are
 * per-program symbols, looked up by name (ctypes.c_void_p.in_dll). */

/* ---- profiling (the reference's `anvil run --profile`, aarch64.py:382-402) -------------------- */
void anvil_profile_enable(int on);        /* HIP events around every launch while on */
void anvil_profile_reset(void);
int anvil_profile_count(void);            /* launch sites: one per generated kernel */
const char *anvil_profile_label(int site);
double anvil_profile_ms(int site);        /* total device time */
long anvil_profile_calls(int site);
double anvil_profile_flops(int site);     /* algorithmic FLOPs of one launch (cost.py:22-37 rules) */
double anvil_profile_bytes(int site);     /* algorithmic bytes of one launch (cost.py:40-52 rules) */
const char *anvil_profile_where(int site); /* the row text of the --profile table: name, label, file:line */
void anvil_profile_print(void);          /* the --profile table on stdout (runtime.s:1592-1671 form) */

/* ---- loop marks: a device event at the start of each iteration of the loops whose counter has
 * this name, for timing exactly K iterations. No counterpart in the reference. ---------------- */
void anvil_marks_select(const char *counter_name);
int anvil_marks_window(int first, int last);   /* events only at these two iterations; -1 if not 0 <= first <= last */
int anvil_marks_count(void);
double anvil_marks_elapsed_ms(int from_mark, int to_mark);   /* -1 where a mark has no event */

/* ---- inspection ------------------------------------------------------------------------------ */
/* Copy buffer `id` (its ir.Buffer.id) into dst; returns the bytes copied, -1 if the library holds
 * no such buffer, -2 if dst is too small. Waits for the device. */
int anvil_buffer_read(int id, void *dst, long long bytes);
long long anvil_arena_bytes(void);          /* the device arena (arena.py:121-144 lifetime sharing) */
long long anvil_arena_unshared_bytes(void); /* what the same buffers would take without sharing */
const char *anvil_target(void);             /* "gfx950" */

#ifdef __cplusplus
}
#endif
#endif
