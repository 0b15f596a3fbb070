// Launch descriptor for the on-device nucleus sampler (sample.hip): the
// reference's top_p_sample (main.py:49-87) -- temperature, repetition penalty
// over a window of recent tokens, top-k(2000) candidates normalised against
// the full vocabulary, top-p cut, multinomial draw -- with every step on the
// GPU and no host synchronisation, so a decode step that samples can be
// captured in a HIP graph.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

struct QhSampleParams {
  const uint16_t* logits;   // [V] bf16
  int V;
  float temperature;        // > 0: logits / temperature (bf16); otherwise unscaled
  float top_p;
  float rep_penalty;        // > 1: penalise the tokens of the recent window
  // Recent window (main.py:1720-1731 keeps the last 50 generated tokens): the
  // new token goes to slot p = *pos_dev + pos_offset (or `pos` without
  // pos_dev); the window is hist[max(lo, p - window) .. p) with lo = *lo_dev
  // (or 0 without lo_dev).  Only slots in [0, hist_len) are read or written:
  // a slot past the end gets no write-back and the window is clipped to it.
  int64_t* hist;            // token history (optional: no penalty, no write-back)
  int hist_len;             // entries in hist
  const int* pos_dev;
  int pos;
  int pos_offset;
  const int* lo_dev;
  int window;               // <= kSampleMaxWindow
  uint64_t seed;
  uint64_t* counter;        // draw counter (device), advanced by one per call
  uint8_t* ws;              // workspace, qh_sample_workspace_bytes(V)
  int64_t* tok_out;         // the sampled token
  const uint16_t* embed;    // optional [V, D] bf16 table: its row of the token -> h
  uint16_t* h;
  int D;
  int64_t* info;            // optional [16] diagnostics (see sample.hip)
};

constexpr int kSampleMaxWindow = 64;

size_t qh_sample_workspace_bytes(int V);
int qh_launch_sample(const QhSampleParams& p, hipStream_t st);
void qh_set_error(const char* fmt, ...);
