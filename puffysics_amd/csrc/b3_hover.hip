/*
 * b3_hover.hip - the PufferLib hover environment around the engine.
 *
 * The task of examples/pufferlib/puffysics_hover/hover_task.h with the
 * environment step of puffysics_hover.h:38-56, for n envs on one stream.
 * The worlds live in a B3Engine; the per-env task state (RNG, tick, episode
 * return, log) lives in device arrays, one element per env.  A reset is a
 * restore to the task's initial world (b3_world_init, one dynamic sphere
 * of radius 0.25 with default shape and damping 0, finalize_mass) followed
 * by the new start height, which is the only world word that depends on
 * the reset's random draw; b3_hover_create checks that on the host.
 * Compiled with the hover capacities (2 bodies, 2 shapes, 4 contacts, 2
 * joints; hover_task.h:4-16).
 */
#define B3_MAX_BODIES 2
#define B3_MAX_SHAPES 2
#define B3_MAX_CONTACTS 4
#define B3_MAX_JOINTS 2
#include <hip/hip_runtime.h>

#include <math.h>
#include <stddef.h>
#include <stdlib.h>
#include <string.h>

#include "b3_hover.h"
#include "b3_setup.h"

struct B3HoverEnvs {
    int device;
    int n;
    B3HoverConfig config;
    B3Engine* engine;
    uint32_t* tiles;
    size_t world_words;
    float *obs, *actions, *rewards, *terminals;  /* the caller's */
    uint32_t* rng;
    int* tick;
    float* ep_return;
    float* log;          /* n * 5: perf, score, episode_return, episode_length, n */
    float* start_y;      /* the next episode's start height */
    unsigned char* reset;
};

namespace {

constexpr int kThreads = 256;
/* the task's body is the first one a fresh world creates */
constexpr int kBody = 0;
constexpr int W_POS_Y = (int)(offsetof(B3World, bodies[kBody].position.y) / 4);
constexpr int W_CENTER_Y = (int)(offsetof(B3World, bodies[kBody].center.y) / 4);
constexpr int W_VEL_Y = (int)(offsetof(B3World, bodies[kBody].lin_vel.y) / 4);
constexpr int W_FORCE = (int)(offsetof(B3World, bodies[kBody].force) / 4);
constexpr int W_INV_MASS = (int)(offsetof(B3World, bodies[kBody].inv_mass) / 4);

/* word k of env i's world in the engine's tiles */
__device__ __forceinline__ uint32_t* word(uint32_t* tiles, size_t ww, int i, int k) {
    return tiles + ((size_t)(i >> 6) * ww + (size_t)k) * 64 + (i & 63);
}
__device__ __forceinline__ float getf(uint32_t* tiles, size_t ww, int i, int k) {
    return __builtin_bit_cast(float, *word(tiles, ww, i, k));
}
__device__ __forceinline__ void setf(uint32_t* tiles, size_t ww, int i, int k, float v) {
    *word(tiles, ww, i, k) = __builtin_bit_cast(uint32_t, v);
}

/* hover_reset's draw (hover_task.h:46-48): the next RNG state and the start
 * height target + jitter. */
__host__ __device__ __forceinline__ uint32_t next_rng(uint32_t r) { return r * 1664525u + 1013904223u; }
__host__ __device__ __forceinline__ float start_height(float target, uint32_t r) {
    float jitter = (float)(r >> 8) * (1.0f / 16777216.0f) - 0.5f;
    return target + jitter;
}

/* hover_apply_action (hover_task.h:68-73) through b3_apply_force. */
__global__ __launch_bounds__(kThreads) void hk_action(uint32_t* tiles, size_t ww, int n, const float* actions,
        float thrust) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float a = actions[i];
    float level = a >= 1.5f ? 2.0f : (a >= 0.5f ? 1.0f : 0.0f);
    float fy = level * thrust / getf(tiles, ww, i, W_INV_MASS);
    setf(tiles, ww, i, W_FORCE, getf(tiles, ww, i, W_FORCE) + 0.0f);
    setf(tiles, ww, i, W_FORCE + 1, getf(tiles, ww, i, W_FORCE + 1) + fy);
    setf(tiles, ww, i, W_FORCE + 2, getf(tiles, ww, i, W_FORCE + 2) + 0.0f);
}

/* After b3_step: tick, hover_reward, hover_terminal (hover_task.h:81-92),
 * the episode return and log, and for envs that are done the draw of the
 * next start height (puffysics_hover.h:40-52). */
__global__ __launch_bounds__(kThreads) void hk_reward(uint32_t* tiles, size_t ww, int n, B3HoverConfig cfg,
        int* tick, float* ep_return, float* log, uint32_t* rng, float* start_y, unsigned char* reset, float* rewards,
        float* terminals) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    int t = tick[i] + 1;
    float y = getf(tiles, ww, i, W_POS_Y);
    float vy = getf(tiles, ww, i, W_VEL_Y);
    float error = fabsf(y - cfg.target_height);
    float e = error + 0.1f * fabsf(vy);
    float reward = 1.0f - (e < 2.0f ? e : 2.0f);
    int done = !isfinite(y) || fabsf(y - cfg.target_height) > 3.0f || t >= cfg.horizon;
    float ret = ep_return[i] + reward;
    if (done) {
        float* lg = log + (size_t)i * 5;
        lg[0] += t >= cfg.horizon;
        lg[1] += ret;
        lg[2] += ret;
        lg[3] += (float)t;
        lg[4] += 1;
        uint32_t r = next_rng(rng[i]);
        rng[i] = r;
        start_y[i] = start_height(cfg.target_height, r);
        t = 0;
        ret = 0;
    }
    tick[i] = t;
    ep_return[i] = ret;
    reset[i] = (unsigned char)done;
    rewards[i] = reward;
    terminals[i] = (float)done;
}

/* hover_reset for every env (hover_env_reset, puffysics_hover.h:31-36). */
__global__ __launch_bounds__(kThreads) void hk_reset_all(int n, B3HoverConfig cfg, int* tick, float* ep_return,
        uint32_t* rng, float* start_y, unsigned char* reset, float* rewards, float* terminals) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    uint32_t r = next_rng(rng[i]);
    rng[i] = r;
    start_y[i] = start_height(cfg.target_height, r);
    tick[i] = 0;
    ep_return[i] = 0.0f;
    reset[i] = 1;
    rewards[i] = 0.0f;
    terminals[i] = 0.0f;
}

/* Reset envs take their start height; then hover_observe
 * (hover_task.h:75-79) for every env. */
__global__ __launch_bounds__(kThreads) void hk_observe(uint32_t* tiles, size_t ww, int n, B3HoverConfig cfg,
        const int* tick, const float* start_y, const unsigned char* reset, float* obs) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    if (reset[i]) {
        setf(tiles, ww, i, W_POS_Y, start_y[i]);
        setf(tiles, ww, i, W_CENTER_Y, start_y[i]);
    }
    obs[(size_t)i * 3] = getf(tiles, ww, i, W_POS_Y) - cfg.target_height;
    obs[(size_t)i * 3 + 1] = getf(tiles, ww, i, W_VEL_Y);
    obs[(size_t)i * 3 + 2] = (float)tick[i] / (float)cfg.horizon;
}

/* hover_reset's world for the draw r (hover_task.h:44-60). */
void task_world(B3World* w, const B3HoverConfig& cfg, uint32_t r, int* body) {
    b3_world_init(w);
    B3BodyDef def = b3_default_body();
    def.type = B3_DYNAMIC;
    def.position = b3_v(0, start_height(cfg.target_height, r), 0);
    def.linear_damping = 0;
    *body = b3_create_body(w, &def);
    B3ShapeDef shape = b3_default_shape();
    b3_create_sphere(w, *body, b3_v(0, 0, 0), 0.25f, &shape);
    b3_finalize_mass(w, *body);
}

/* Two draws' worlds differ only in the start height words, which hold the
 * start height itself: what makes a reset a restore plus one word pair. */
bool reset_is_restore(const B3HoverConfig& cfg) {
    B3World* a = (B3World*)calloc(1, sizeof(B3World));
    B3World* b = (B3World*)calloc(1, sizeof(B3World));
    bool ok = a && b;
    if (ok) {
        uint32_t ra = next_rng(1u), rb = next_rng(ra);
        int ba, bb;
        task_world(a, cfg, ra, &ba);
        task_world(b, cfg, rb, &bb);
        ok = ba == kBody && bb == kBody;
        const uint32_t* wa = (const uint32_t*)a;
        const uint32_t* wb = (const uint32_t*)b;
        for (size_t k = 0; ok && k < sizeof(B3World) / 4; k++) {
            if ((int)k == W_POS_Y || (int)k == W_CENTER_Y) {
                float ya = start_height(cfg.target_height, ra), yb = start_height(cfg.target_height, rb);
                ok = wa[k] == __builtin_bit_cast(uint32_t, ya) && wb[k] == __builtin_bit_cast(uint32_t, yb);
            } else {
                ok = wa[k] == wb[k];
            }
        }
    }
    free(a);
    free(b);
    return ok;
}

unsigned grid(int n) { return (unsigned)((n + kThreads - 1) / kThreads); }

}  // namespace

extern "C" {

B3HoverConfig b3_hover_default_config(void) {
    B3HoverConfig c;
    c.target_height = 2.0f;
    c.thrust = 10.0f;
    c.dt = 1.0f / 60.0f;
    c.substeps = 4;
    c.horizon = 256;
    return c;
}

hipError_t b3_hover_destroy(B3HoverEnvs* h) {
    if (!h) return hipSuccess;
    hipError_t first = b3_engine_destroy(h->engine);
    void* bufs[6] = {h->rng, h->tick, h->ep_return, h->log, h->start_y, h->reset};
    for (void* p : bufs) {
        if (!p) continue;
        hipError_t err = hipFree(p);
        if (first == hipSuccess) first = err;
    }
    free(h);
    return first;
}

hipError_t b3_hover_create(B3HoverEnvs** out, int n, B3HoverConfig cfg, uint32_t seed, float* obs, float* actions,
        float* rewards, float* terminals) {
    if (!out) return hipErrorInvalidValue;
    *out = NULL;
    if (n <= 0 || !obs || !actions || !rewards || !terminals || !isfinite(cfg.target_height) || !isfinite(cfg.thrust)
            || !isfinite(cfg.dt) || cfg.dt < 0.0f || cfg.substeps < 1 || cfg.horizon < 1)
        return hipErrorInvalidValue;
    if (!reset_is_restore(cfg)) return hipErrorNotSupported;
    B3HoverEnvs* h = (B3HoverEnvs*)calloc(1, sizeof(B3HoverEnvs));
    if (!h) return hipErrorOutOfMemory;
    h->n = n;
    h->config = cfg;
    h->obs = obs;
    h->actions = actions;
    h->rewards = rewards;
    h->terminals = terminals;
    hipError_t err = hipGetDevice(&h->device);
    /* hover_init per env (hover_task.h:62-66, puffysics_hover.cu:41) */
    B3World* worlds = (B3World*)calloc((size_t)n, sizeof(B3World));
    uint32_t* rng = (uint32_t*)malloc((size_t)n * sizeof(uint32_t));
    if (!worlds || !rng) err = hipErrorOutOfMemory;
    if (err == hipSuccess) {
        for (int i = 0; i < n; i++) {
            rng[i] = next_rng(seed + (uint32_t)i * 747796405u);
            int body;
            task_world(&worlds[i], cfg, rng[i], &body);
        }
        B3Batch batch = {worlds, sizeof(B3World), 0, n};
        err = b3_engine_create(&h->engine, batch, b3_config_signature());
    }
    if (err == hipSuccess) {
        /* every env restores to the first env's world (its start height is
         * overwritten after each restore) */
        for (int i = 1; i < n; i++) memcpy(&worlds[i], &worlds[0], sizeof(B3World));
        err = b3_engine_set_snapshots(h->engine, worlds);
    }
    void* tiles = NULL;
    if (err == hipSuccess) err = b3_engine_device_view(h->engine, &tiles, &h->world_words);
    h->tiles = (uint32_t*)tiles;
    if (err == hipSuccess) err = hipMalloc((void**)&h->rng, (size_t)n * sizeof(uint32_t));
    if (err == hipSuccess) err = hipMalloc((void**)&h->tick, (size_t)n * sizeof(int));
    if (err == hipSuccess) err = hipMalloc((void**)&h->ep_return, (size_t)n * sizeof(float));
    if (err == hipSuccess) err = hipMalloc((void**)&h->log, (size_t)n * 5 * sizeof(float));
    if (err == hipSuccess) err = hipMalloc((void**)&h->start_y, (size_t)n * sizeof(float));
    if (err == hipSuccess) err = hipMalloc((void**)&h->reset, (size_t)n);
    if (err == hipSuccess) err = hipMemcpy(h->rng, rng, (size_t)n * sizeof(uint32_t), hipMemcpyHostToDevice);
    if (err == hipSuccess) err = hipMemset(h->tick, 0, (size_t)n * sizeof(int));
    if (err == hipSuccess) err = hipMemset(h->ep_return, 0, (size_t)n * sizeof(float));
    if (err == hipSuccess) err = hipMemset(h->log, 0, (size_t)n * 5 * sizeof(float));
    if (err == hipSuccess) err = hipMemset(h->reset, 0, (size_t)n);
    if (err == hipSuccess) err = hipDeviceSynchronize();
    free(worlds);
    free(rng);
    if (err != hipSuccess) {
        (void)b3_hover_destroy(h);
        return err;
    }
    *out = h;
    return hipSuccess;
}

hipError_t b3_hover_reset(B3HoverEnvs* h, hipStream_t stream) {
    if (!h) return hipErrorInvalidValue;
    hk_reset_all<<<grid(h->n), kThreads, 0, stream>>>(h->n, h->config, h->tick, h->ep_return, h->rng, h->start_y,
        h->reset, h->rewards, h->terminals);
    hipError_t err = hipGetLastError();
    if (err == hipSuccess) err = b3_batch_restore_gpu(h->engine, NULL, stream);
    if (err != hipSuccess) return err;
    hk_observe<<<grid(h->n), kThreads, 0, stream>>>(h->tiles, h->world_words, h->n, h->config, h->tick, h->start_y,
        h->reset, h->obs);
    return hipGetLastError();
}

hipError_t b3_hover_step(B3HoverEnvs* h, hipStream_t stream) {
    if (!h) return hipErrorInvalidValue;
    hk_action<<<grid(h->n), kThreads, 0, stream>>>(h->tiles, h->world_words, h->n, h->actions, h->config.thrust);
    hipError_t err = hipGetLastError();
    if (err == hipSuccess) err = b3_batch_step_gpu(h->engine, h->config.dt, h->config.substeps, NULL, NULL, stream);
    if (err != hipSuccess) return err;
    hk_reward<<<grid(h->n), kThreads, 0, stream>>>(h->tiles, h->world_words, h->n, h->config, h->tick, h->ep_return,
        h->log, h->rng, h->start_y, h->reset, h->rewards, h->terminals);
    err = hipGetLastError();
    if (err == hipSuccess) err = b3_batch_restore_gpu(h->engine, h->reset, stream);
    if (err != hipSuccess) return err;
    hk_observe<<<grid(h->n), kThreads, 0, stream>>>(h->tiles, h->world_words, h->n, h->config, h->tick, h->start_y,
        h->reset, h->obs);
    return hipGetLastError();
}

hipError_t b3_hover_log(B3HoverEnvs* h, B3HoverLog* out, hipStream_t stream) {
    if (!h || !out) return hipErrorInvalidValue;
    float* host = (float*)malloc((size_t)h->n * 5 * sizeof(float));
    if (!host) return hipErrorOutOfMemory;
    hipError_t err = hipMemcpyAsync(host, h->log, (size_t)h->n * 5 * sizeof(float), hipMemcpyDeviceToHost, stream);
    if (err == hipSuccess) err = hipStreamSynchronize(stream);
    if (err == hipSuccess) {
        float s[5] = {0, 0, 0, 0, 0};
        for (int i = 0; i < h->n; i++)
            for (int k = 0; k < 5; k++) s[k] += host[(size_t)i * 5 + k];
        out->perf = s[0];
        out->score = s[1];
        out->episode_return = s[2];
        out->episode_length = s[3];
        out->n = s[4];
    }
    free(host);
    return err;
}

B3Engine* b3_hover_engine(B3HoverEnvs* h) { return h ? h->engine : NULL; }

}  // extern "C"
