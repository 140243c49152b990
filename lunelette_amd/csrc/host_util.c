/* Host-side pieces of the forward path: YaRN tables, the query factor, and the
 * seeded synthetic-tensor generator. */
#include "lunelette_kernels.h"

#include <math.h>
#include <pthread.h>
#include <string.h>
#include <unistd.h>

/* YaRN cos/sin for one position (src/metal_yarn.c:8-33): correction bounds
 * floor/ceil of dim*ln(orig/(beta*2pi))/(2 ln theta) in double, with
 * beta_fast 32 and beta_slow 1, original context 16384, theta 1e6, factor 16,
 * mscale 1; then per half-dimension j in FP32 with contraction off, keeping
 * the interpolation written as inv_interp*(1-ext) + inv_extrap*ext. */
int lh_yarn(uint32_t position, float cosine[128], float sine[128])
{
    if (position >= 262144u || !cosine || !sine) {
        return -1;
    }
    const double two_pi = 2.0 * 3.14159265358979323846;
    const double denominator = 2.0 * log(1e6);
    const float low = (float)floor(128.0 * log(16384.0 / (32.0 * two_pi)) / denominator);
    const float high = (float)ceil(128.0 * log(16384.0 / two_pi) / denominator);
    for (int j = 0; j < 64; j++) {
        const float frequency = powf(1000000.0f, (float)(2 * j) / 128.0f);
        const float ramp = fminf(1.0f, fmaxf(0.0f, ((float)j - low) / (high - low)));
        const float extrapolation = 1.0f - ramp;
        const float inverse = (1.0f / (16.0f * frequency)) * (1.0f - extrapolation) +
            (1.0f / frequency) * extrapolation;
        const float angle = inverse * (float)position;
        const float c = cosf(angle), s = sinf(angle);
        cosine[j] = cosine[j + 64] = c;
        sine[j] = sine[j + 64] = s;
    }
    return 0;
}

float lh_query_factor(uint32_t position)
{
    return 1.0f + 0.1f * logf(1.0f + (float)(position / 16384u));
}

/* ---- synthetic tensors: counter-based splitmix64 ---- */

static inline uint64_t mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}

static inline uint64_t stream_base(uint64_t seed, uint32_t tensor)
{
    return mix64(seed * 0x9e3779b97f4a7c15ULL + ((uint64_t)tensor + 1) * 0xd1b54a32d192ed03ULL);
}

static inline uint64_t element_hash(uint64_t base, uint64_t index)
{
    return mix64(base + index * 0x9e3779b97f4a7c15ULL);
}

/* Normal sample by Box-Muller (cosine branch) in double from two hashes. */
static inline double normal_at(uint64_t base, uint64_t index)
{
    uint64_t a = element_hash(base, 2 * index), b = element_hash(base, 2 * index + 1);
    double u1 = ((double)(a >> 11) + 0.5) * (1.0 / 9007199254740992.0);
    double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586476925286766559 * u2);
}

static uint16_t bf16_round(float value)
{
    uint32_t word;
    memcpy(&word, &value, sizeof word);
    word += 0x7fffu + ((word >> 16) & 1u);
    return (uint16_t)(word >> 16);
}

typedef struct {
    int kind; /* 0 fp8, 1 normal f32, 2 normal bf16 */
    uint64_t base, offset;
    float mean, std;
    void *out;
    size_t begin, end;
} synth_job;

static void synth_range(const synth_job *job)
{
    for (size_t i = job->begin; i < job->end; i++) {
        uint64_t index = job->offset + i;
        if (job->kind == 0) {
            /* k uniform in [0,254); skipping 127 excludes 0x7f and 0xff. */
            uint32_t k = (uint32_t)((element_hash(job->base, index) >> 32) % 254u);
            ((uint8_t *)job->out)[i] = (uint8_t)(k + (k >= 127u));
        } else {
            float value = (float)(job->mean + job->std * normal_at(job->base, index));
            if (job->kind == 1) {
                ((float *)job->out)[i] = value;
            } else {
                ((uint16_t *)job->out)[i] = bf16_round(value);
            }
        }
    }
}

static void *synth_worker(void *arg)
{
    synth_range((const synth_job *)arg);
    return NULL;
}

static void synth_parallel(synth_job job, size_t n)
{
    long cpus = sysconf(_SC_NPROCESSORS_ONLN);
    size_t workers = cpus > 16 ? 16 : (cpus < 1 ? 1 : (size_t)cpus);
    if (n < ((size_t)1 << 20)) {
        workers = 1;
    }
    pthread_t threads[16];
    synth_job jobs[16];
    size_t started = 0;
    for (size_t w = 0; w < workers; w++) {
        jobs[w] = job;
        jobs[w].begin = n * w / workers;
        jobs[w].end = n * (w + 1) / workers;
        if (w + 1 < workers && pthread_create(&threads[w], NULL, synth_worker, &jobs[w]) == 0) {
            started++;
        } else if (w + 1 < workers) {
            synth_range(&jobs[w]);
            threads[w] = 0;
        }
    }
    synth_range(&jobs[workers - 1]);
    for (size_t w = 0; w + 1 < workers; w++) {
        if (threads[w]) {
            pthread_join(threads[w], NULL);
        }
    }
    (void)started;
}

void lh_synth_fp8(uint64_t seed, uint32_t tensor, uint64_t offset, uint8_t *out, size_t n)
{
    synth_job job = {0, stream_base(seed, tensor), offset, 0, 0, out, 0, 0};
    synth_parallel(job, n);
}

void lh_synth_normal_f32(uint64_t seed, uint32_t tensor, uint64_t offset, float mean, float std,
    float *out, size_t n)
{
    synth_job job = {1, stream_base(seed, tensor), offset, mean, std, out, 0, 0};
    synth_parallel(job, n);
}

void lh_synth_normal_bf16(uint64_t seed, uint32_t tensor, uint64_t offset, float mean, float std,
    uint16_t *out, size_t n)
{
    synth_job job = {2, stream_base(seed, tensor), offset, mean, std, out, 0, 0};
    synth_parallel(job, n);
}

float lh_synth_scale(uint64_t seed, uint32_t tensor)
{
    uint64_t h = element_hash(stream_base(seed, tensor ^ 0x5ca1e000u), 0);
    double u = (double)(h >> 11) * (1.0 / 9007199254740992.0);
    /* Truncate to BF16 inside [0.01, 0.02]: both ends are interior to the
     * range after truncation. */
    float value = (float)(0.0101 + 0.0098 * u);
    uint32_t word;
    memcpy(&word, &value, sizeof word);
    word &= 0xffff0000u;
    memcpy(&value, &word, sizeof value);
    return value;
}

void lh_synth_tokens(uint64_t seed, uint32_t stream_id, int64_t *out, size_t n)
{
    uint64_t base = stream_base(seed, 0x70000000u + stream_id);
    for (size_t i = 0; i < n; i++) {
        out[i] = (int64_t)(element_hash(base, i) >> 47); /* 17 bits: [0, 131072) */
    }
}
