/* pt_queue.c -- queue-fed serving of the device-resident decoder (include/ptd.h, ptd_queue_*).
 *
 * The reference's server (runtime/v21/src/main_v21_serve.c) runs persistent workers, each with
 * its own context opened once (:281-335), popping jobs from one bounded queue ordered earliest-
 * deadline-first and stable among equal deadlines (:129-160); a streamed reply decodes a short
 * first window for fast first audio, then longer windows (:210-264).  Here the same model runs
 * on the decoder API: each worker owns a pt_ctx (stream + arena) over one shared ptd_model, a
 * job is one ptd_decode or one windowed decode whose first window is completed and timed before
 * the rest runs batched, and callers wait for or poll their job's completion. */
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#include "pt_dev_internal.h"
#include "ptd.h"

#define QUEUE_MAX_WORKERS 256
#define QUEUE_DEFAULT_CAP 64   /* the reference's MAX_QUEUE (main_v21_serve.c:56) */

enum { SLOT_FREE = 0, SLOT_QUEUED, SLOT_RUNNING, SLOT_DONE };

typedef struct qjob {
  int64_t id;
  int state;
  ptd_job job;
  ptd_job_status st;
  struct qjob *next;   /* EDF list link while queued */
} qjob;

typedef struct {
  struct ptd_queue *q;
  int i;
} qworker_arg;

struct ptd_queue {
  const ptd_model *m;
  int nw, cap, nthreads;
  size_t arena_bytes;
  pt_ctx *ctx;
  void *ballast[PTDI_PLACE_MAX_BALLAST];   /* see ptdi_place_streams */
  pthread_t *th;
  qworker_arg *args;
  qjob *slots;
  qjob *head;          /* queued jobs, ascending deadline, submission order among equals */
  int64_t next_id, next_order;
  int hold, closing;
  pthread_mutex_t mu;
  pthread_cond_t cv_work, cv_done;
};

double ptd_now_ms(void) { return ptdi_now_ms(); }

static int run_job(pt_ctx *c, const ptd_model *m, const ptd_job *j, double *t_first) {
  int rc;
  if (j->win > 0) {
    rc = ptdi_decode_windows(c, m, j->z, j->T, j->win_first, j->win, j->ctx, j->wav, t_first);
  } else {
    rc = ptd_decode(c, m, j->z, j->T, 1, j->wav);
  }
  if (ptdi_wait(c)) rc = -1;
  return rc;
}

static void *qworker(void *p) {
  qworker_arg *a = (qworker_arg *) p;
  struct ptd_queue *q = a->q;
  pt_ctx *c = &q->ctx[a->i];
  if (ptk_init()) PT_LOG("queue worker %d: %s", a->i, ptk_last_error());
  pthread_mutex_lock(&q->mu);
  for (;;) {
    while (!q->head || (q->hold && !q->closing)) {
      if (!q->head && q->closing) break;
      pthread_cond_wait(&q->cv_work, &q->mu);
    }
    if (!q->head) break;   /* closing and nothing left */
    qjob *j = q->head;
    q->head = j->next;
    j->next = NULL;
    j->state = SLOT_RUNNING;
    j->st.order = q->next_order++;
    j->st.worker = a->i;
    j->st.t_start = ptdi_now_ms();
    const ptd_job job = j->job;
    pthread_mutex_unlock(&q->mu);

    pt_v21_cuda_active(1);
    double t_first = -1.0;
    const int rc = run_job(c, q->m, &job, job.win > 0 ? &t_first : NULL);
    const double t_end = ptdi_now_ms();
    pt_v21_cuda_active(-1);

    pthread_mutex_lock(&q->mu);
    j->st.rc = rc;
    j->st.t_end = t_end;
    j->st.t_first = t_first >= 0.0 && rc == 0 ? t_first : t_end;
    j->state = SLOT_DONE;
    pthread_cond_broadcast(&q->cv_done);
  }
  pthread_mutex_unlock(&q->mu);
  return NULL;
}

static void queue_free(struct ptd_queue *q) {
  if (q->ctx)
    for (int i = 0; i < q->nw; i++)
      if (q->ctx[i].use_cuda) pt_v21_cuda_shutdown(&q->ctx[i]);
  ptdi_place_release(q->ballast);
  pthread_mutex_destroy(&q->mu);
  pthread_cond_destroy(&q->cv_work);
  pthread_cond_destroy(&q->cv_done);
  free(q->ctx);
  free(q->th);
  free(q->args);
  free(q->slots);
  free(q);
}

static void queue_stop(struct ptd_queue *q) {
  pthread_mutex_lock(&q->mu);
  q->closing = 1;
  q->hold = 0;
  pthread_cond_broadcast(&q->cv_work);
  pthread_mutex_unlock(&q->mu);
  for (int i = 0; i < q->nthreads; i++) pthread_join(q->th[i], NULL);
  q->nthreads = 0;
}

ptd_queue *ptd_queue_create(const ptd_model *m, int nworkers, size_t arena_bytes, int capacity) {
  if (!m || nworkers < 1 || nworkers > QUEUE_MAX_WORKERS) return NULL;
  if (capacity <= 0) capacity = QUEUE_DEFAULT_CAP;
  struct ptd_queue *q = calloc(1, sizeof *q);
  if (!q) return NULL;
  q->m = m;
  q->nw = nworkers;
  q->cap = capacity;
  q->arena_bytes = arena_bytes;
  pthread_mutex_init(&q->mu, NULL);
  pthread_cond_init(&q->cv_work, NULL);
  pthread_cond_init(&q->cv_done, NULL);
  q->ctx = calloc((size_t) nworkers, sizeof(pt_ctx));
  q->th = calloc((size_t) nworkers, sizeof(pthread_t));
  q->args = calloc((size_t) nworkers, sizeof(qworker_arg));
  q->slots = calloc((size_t) capacity, sizeof(qjob));
  if (!q->ctx || !q->th || !q->args || !q->slots) {
    queue_free(q);
    return NULL;
  }
  for (int i = 0; i < nworkers; i++) {
    if (ptdi_ctx_init(&q->ctx[i], arena_bytes, 0)) {
      PT_LOG("ptd_queue_create: context %d of %d failed", i, nworkers);
      queue_free(q);
      return NULL;
    }
  }
  if (ptdi_place_streams(q->ctx, nworkers, q->ballast)) {
    queue_free(q);
    return NULL;
  }
  /* after every worker's stream: a worker's first long-form job then makes no streams */
  for (int i = 0; i < nworkers; i++) ptdi_aux_prepare(&q->ctx[i]);
  for (int i = 0; i < nworkers; i++) {
    q->args[i] = (qworker_arg){q, i};
    if (pthread_create(&q->th[i], NULL, qworker, &q->args[i])) {
      PT_LOG("ptd_queue_create: worker thread %d failed", i);
      queue_stop(q);
      queue_free(q);
      return NULL;
    }
    q->nthreads++;
  }
  return q;
}

void ptd_queue_destroy(ptd_queue *q) {
  if (!q) return;
  queue_stop(q);
  queue_free(q);
}

void ptd_queue_hold(ptd_queue *q, int hold) {
  if (!q) return;
  pthread_mutex_lock(&q->mu);
  q->hold = hold != 0;
  if (!q->hold) pthread_cond_broadcast(&q->cv_work);
  pthread_mutex_unlock(&q->mu);
}

int64_t ptd_queue_submit(ptd_queue *q, const ptd_job *job) {
  if (!q || !job || !job->z || !job->wav || job->T < 1) return -1;
  /* a job the workers' arenas cannot hold is refused here, not failed later */
  size_t need;
  if (job->win > 0) {
    need = ptd_windows2_arena_bytes(job->T, job->win_first, job->win, job->ctx);
    if (need == 0) return -1;   /* malformed window schedule */
  } else {
    need = ptd_decode_arena_bytes(job->T, 1);
  }
  if (need > q->arena_bytes) {
    PT_LOG("ptd_queue_submit: a job of T %lld needs %zu MiB of arena; workers have %zu MiB",
           (long long) job->T, need >> 20, q->arena_bytes >> 20);
    return -1;
  }
  pthread_mutex_lock(&q->mu);
  qjob *j = NULL;
  if (!q->closing)
    for (int i = 0; i < q->cap && !j; i++)
      if (q->slots[i].state == SLOT_FREE) j = &q->slots[i];
  if (!j) {
    pthread_mutex_unlock(&q->mu);
    return -1;   /* full (or closing): the reference answers 503 */
  }
  memset(j, 0, sizeof *j);
  j->id = q->next_id++;
  j->job = *job;
  if (job->win > 0) ptdi_serve_widths(&j->job.win_first, &j->job.win, j->job.ctx);
  j->state = SLOT_QUEUED;
  j->st.order = -1;
  j->st.worker = -1;
  j->st.t_submit = ptdi_now_ms();
  qjob **pp = &q->head;
  while (*pp && (*pp)->job.deadline_ms <= job->deadline_ms) pp = &(*pp)->next;
  j->next = *pp;
  *pp = j;
  const int64_t id = j->id;
  pthread_cond_signal(&q->cv_work);
  pthread_mutex_unlock(&q->mu);
  return id;
}

static qjob *find(struct ptd_queue *q, int64_t id) {
  for (int i = 0; i < q->cap; i++)
    if (q->slots[i].state != SLOT_FREE && q->slots[i].id == id) return &q->slots[i];
  return NULL;
}

int ptd_queue_poll(ptd_queue *q, int64_t id, ptd_job_status *st) {
  if (!q) return -1;
  pthread_mutex_lock(&q->mu);
  qjob *j = find(q, id);
  int r = -1;
  if (j) {
    r = j->state == SLOT_DONE;
    if (r) {
      if (st) *st = j->st;
      j->state = SLOT_FREE;
    }
  }
  pthread_mutex_unlock(&q->mu);
  return r;
}

int ptd_queue_wait(ptd_queue *q, int64_t id, ptd_job_status *st) {
  if (!q) return -1;
  pthread_mutex_lock(&q->mu);
  qjob *j = find(q, id);
  if (!j) {
    pthread_mutex_unlock(&q->mu);
    return -1;
  }
  /* another waiter on the same id may take the result (and the slot a new job) first */
  while (j->id == id && (j->state == SLOT_QUEUED || j->state == SLOT_RUNNING))
    pthread_cond_wait(&q->cv_done, &q->mu);
  int r = -1;
  if (j->id == id && j->state == SLOT_DONE) {
    if (st) *st = j->st;
    j->state = SLOT_FREE;
    r = 0;
  }
  pthread_mutex_unlock(&q->mu);
  return r;
}
