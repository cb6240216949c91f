/*
 * CPU baseline timings for the KV-cache + decode-attention path.
 *
 * TEST/BENCH INFRASTRUCTURE ONLY: bench.py's cpu_baseline leg and tests/ use
 * it; the product library never links or calls it.
 *
 * What is timed is the oracle's restatement of the reference host attention
 * (tests/test_flash_attention.cu:124-172, applied to the decode row through
 * the page table as oracle_decode_attention does) plus the reference append
 * (src/gemma4_kv_cache.cu:25-54) and ring bookkeeping
 * (src/gemma4_kv_cache.cu:108-146), either on one thread (the reference's
 * own single-threaded host reference) or split over (sequence, KV head)
 * tasks on a pool of host threads. Timing uses CLOCK_MONOTONIC around the
 * compute only; inputs are generated before the clock starts.
 */
#define _GNU_SOURCE
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

static double now_seconds(void) {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

/* ---- seeded N(0,1) bf16 fill ------------------------------------------- */

static uint64_t splitmix64(uint64_t *x) {
  uint64_t z = (*x += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

/* Uniform in (0, 1]: 53 random bits. */
static double unit_open(uint64_t *state) {
  return ((double)(splitmix64(state) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
}

enum { kFillChunk = 1 << 20 };

typedef struct {
  uint16_t *dst;
  int64_t n;
  uint64_t seed;
  float scale;
  atomic_long next;
} FillJob;

/* Chunk c of the array is generated from its own stream (seed, c), so the
 * values do not depend on the thread count. Box-Muller pairs. */
static void fill_chunk(FillJob *job, int64_t c) {
  uint64_t state = job->seed ^ (0xD1B54A32D192ED03ull * (uint64_t)(c + 1));
  const int64_t begin = c * kFillChunk;
  const int64_t end = begin + kFillChunk < job->n ? begin + kFillChunk : job->n;
  for (int64_t i = begin; i < end; i += 2) {
    const double r = sqrt(-2.0 * log(unit_open(&state)));
    const double a = 6.283185307179586 * unit_open(&state);
    job->dst[i] = oracle_f32_to_bf16((float)(r * cos(a)) * job->scale);
    if (i + 1 < end) job->dst[i + 1] = oracle_f32_to_bf16((float)(r * sin(a)) * job->scale);
  }
}

static void *fill_worker(void *arg) {
  FillJob *job = (FillJob *)arg;
  const int64_t chunks = (job->n + kFillChunk - 1) / kFillChunk;
  for (;;) {
    const int64_t c = atomic_fetch_add(&job->next, 1);
    if (c >= chunks) break;
    fill_chunk(job, c);
  }
  return NULL;
}

void oracle_fill_normal_bf16(uint16_t *dst, int64_t n, uint64_t seed, float scale,
                             int32_t threads) {
  FillJob job;
  job.dst = dst;
  job.n = n;
  job.seed = seed;
  job.scale = scale;
  atomic_init(&job.next, 0);
  if (threads < 1) threads = 1;
  pthread_t *t = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)threads);
  for (int32_t i = 1; i < threads; ++i) pthread_create(&t[i], NULL, fill_worker, &job);
  fill_worker(&job);
  for (int32_t i = 1; i < threads; ++i) pthread_join(t[i], NULL);
  free(t);
}

/* ---- a persistent pool of host threads -------------------------------- */

typedef struct Pool Pool;
typedef void (*TaskFn)(void *ctx, int32_t task, int32_t worker);

typedef struct {
  Pool *pool;
  int32_t id;
} WorkerArg;

struct Pool {
  int32_t threads;
  pthread_t *handles;
  WorkerArg *args;
  pthread_barrier_t start, done;
  TaskFn fn;
  void *ctx;
  int32_t tasks;
  atomic_int next;
  int quit;
};

static void pool_drain(Pool *p, int32_t worker) {
  for (;;) {
    const int32_t task = atomic_fetch_add(&p->next, 1);
    if (task >= p->tasks) break;
    p->fn(p->ctx, task, worker);
  }
}

static void *pool_worker(void *arg) {
  WorkerArg *a = (WorkerArg *)arg;
  Pool *p = a->pool;
  for (;;) {
    pthread_barrier_wait(&p->start);
    if (p->quit) break;
    pool_drain(p, a->id);
    pthread_barrier_wait(&p->done);
  }
  return NULL;
}

static void pool_init(Pool *p, int32_t threads) {
  memset(p, 0, sizeof(*p));
  p->threads = threads < 1 ? 1 : threads;
  if (p->threads == 1) return;
  p->handles = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)p->threads);
  p->args = (WorkerArg *)malloc(sizeof(WorkerArg) * (size_t)p->threads);
  pthread_barrier_init(&p->start, NULL, (unsigned)p->threads);
  pthread_barrier_init(&p->done, NULL, (unsigned)p->threads);
  for (int32_t i = 1; i < p->threads; ++i) {
    p->args[i].pool = p;
    p->args[i].id = i;
    pthread_create(&p->handles[i], NULL, pool_worker, &p->args[i]);
  }
}

/* Runs fn(ctx, task, worker) for task = 0..tasks-1 on the pool (the caller
 * is worker 0) and returns when all are done. */
static void pool_run(Pool *p, TaskFn fn, void *ctx, int32_t tasks) {
  p->fn = fn;
  p->ctx = ctx;
  p->tasks = tasks;
  atomic_store(&p->next, 0);
  if (p->threads == 1) {
    pool_drain(p, 0);
    return;
  }
  pthread_barrier_wait(&p->start);
  pool_drain(p, 0);
  pthread_barrier_wait(&p->done);
}

static void pool_free(Pool *p) {
  if (p->threads > 1) {
    p->quit = 1;
    pthread_barrier_wait(&p->start);
    for (int32_t i = 1; i < p->threads; ++i) pthread_join(p->handles[i], NULL);
    pthread_barrier_destroy(&p->start);
    pthread_barrier_destroy(&p->done);
    free(p->handles);
    free(p->args);
  }
}

/* ---- decode attention split over (sequence, KV head) tasks ------------- */

typedef struct {
  float *qf, *acc, *scores;
  int64_t *rows;
} Scratch;

typedef struct {
  uint16_t *out;
  const uint16_t *q, *cache_k, *cache_v;
  const int32_t *page_table, *seq_lengths;
  const OracleKvCacheConfig *c;
  int32_t layer, q_heads;
  float scale;
  Scratch *scratch;  /* [worker] */
} AttnJob;

static void attention_task(void *ctx, int32_t task, int32_t worker) {
  AttnJob *j = (AttnJob *)ctx;
  const int32_t heads = j->c->num_heads;
  const int32_t b = task / heads, kvh = task % heads;
  const int32_t group = j->q_heads / heads;
  Scratch *s = &j->scratch[worker];
  for (int32_t g = 0; g < group; ++g) {
    oracle_decode_attention_row(j->out, j->q, j->cache_k, j->cache_v, j->page_table,
                                j->seq_lengths[b], j->c, j->layer, j->scale, b,
                                kvh * group + g, j->q_heads, s->qf, s->acc, s->scores,
                                s->rows);
  }
}

static Scratch *scratch_alloc(int32_t threads, int32_t head_dim, int32_t max_keys) {
  Scratch *s = (Scratch *)calloc((size_t)threads, sizeof(Scratch));
  const size_t keys = (size_t)(max_keys > 0 ? max_keys : 1);
  for (int32_t i = 0; i < threads; ++i) {
    s[i].qf = (float *)malloc(sizeof(float) * (size_t)head_dim);
    s[i].acc = (float *)malloc(sizeof(float) * (size_t)head_dim);
    s[i].scores = (float *)malloc(sizeof(float) * keys);
    s[i].rows = (int64_t *)malloc(sizeof(int64_t) * keys);
  }
  return s;
}

static void scratch_free(Scratch *s, int32_t threads) {
  for (int32_t i = 0; i < threads; ++i) {
    free(s[i].qf);
    free(s[i].acc);
    free(s[i].scores);
    free(s[i].rows);
  }
  free(s);
}

/* One decode layer-step for `batch` sequences: append each sequence's new
 * K/V row at token_position[b] (reference skip rules), then attend. Returns
 * the seconds the append + attention took. */
double oracle_time_decode_layer(uint16_t *out, const uint16_t *q, uint16_t *cache_k,
                                uint16_t *cache_v, const int32_t *page_table,
                                const int32_t *seq_lengths, const int32_t *token_position,
                                const uint16_t *k_new, const uint16_t *v_new,
                                const OracleKvCacheConfig *c, int32_t layer, float scale,
                                int32_t batch, int32_t q_heads, int32_t threads) {
  int32_t max_keys = 0;
  for (int32_t b = 0; b < batch; ++b)
    if (seq_lengths[b] > max_keys) max_keys = seq_lengths[b];
  Pool pool;
  pool_init(&pool, threads);
  Scratch *scratch = scratch_alloc(pool.threads, c->head_dim, max_keys);
  int32_t *token_batch = (int32_t *)malloc(sizeof(int32_t) * (size_t)(batch > 0 ? batch : 1));
  for (int32_t b = 0; b < batch; ++b) token_batch[b] = b;
  AttnJob job = {out, q, cache_k, cache_v, page_table, seq_lengths, c, layer, q_heads,
                 scale, scratch};
  const double t0 = now_seconds();
  oracle_kv_cache_write(cache_k, cache_v, c, page_table, token_batch, token_position, batch,
                        layer, k_new, v_new);
  pool_run(&pool, attention_task, &job, batch * c->num_heads);
  const double t1 = now_seconds();
  free(token_batch);
  scratch_free(scratch, pool.threads);
  pool_free(&pool);
  return t1 - t0;
}

/* BASELINE config 1: one sliding layer (num_heads x head_dim from `c`, a ring
 * of c->max_pages_per_seq pages of c->page_size), one sequence, `steps`
 * sequential decode steps from an empty cache; step t maps the ring slot of
 * position t (ensure_page), appends q/k/v row t and attends with seq_len
 * t + 1. q/k/v: [steps][q_heads or heads][head_dim] bf16. The cache, page
 * table and slot bookkeeping must come in empty (zeros / -1). `out` receives
 * every step's attention row: [steps][q_heads][head_dim]. Returns seconds,
 * or -1 if a ring slot is refused. */
double oracle_time_config1(uint16_t *out, const uint16_t *q, const uint16_t *k,
                           const uint16_t *v, uint16_t *cache_k, uint16_t *cache_v,
                           int32_t *page_table, int32_t *slot_logical_pages,
                           const OracleKvCacheConfig *c, float scale, int32_t steps,
                           int32_t q_heads, int32_t threads) {
  Pool pool;
  pool_init(&pool, threads);
  Scratch *scratch = scratch_alloc(pool.threads, c->head_dim, steps);
  const int64_t q_row = (int64_t)q_heads * c->head_dim;
  const int64_t kv_row = (int64_t)c->num_heads * c->head_dim;
  const int32_t zero = 0;
  int32_t seq = 0;
  double elapsed = -1.0;
  const double t0 = now_seconds();
  for (int32_t t = 0; t < steps; ++t) {
    if (oracle_kv_cache_ensure_page(page_table, slot_logical_pages, c, 0, t) < 0) goto done;
    oracle_kv_cache_write(cache_k, cache_v, c, page_table, &zero, &t, 1, 0, k + t * kv_row,
                          v + t * kv_row);
    seq = t + 1;
    AttnJob job = {out + t * q_row, q + t * q_row, cache_k, cache_v, page_table, &seq, c, 0,
                   q_heads, scale, scratch};
    pool_run(&pool, attention_task, &job, c->num_heads);
  }
  elapsed = now_seconds() - t0;
done:
  scratch_free(scratch, pool.threads);
  pool_free(&pool);
  return elapsed;
}
