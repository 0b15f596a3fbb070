"""Batch-1 FP8 decode engine for Qwen3.5-shaped hybrid models on one MI355X.

Mirrors the reference engine's public surface (main.py:326-1604,
``QwenEngineFP8Opt``): ``forward(input_ids, past_len, logits_to_keep=1)``
returns bf16 logits of the last position, ``_reset_cache()`` clears the
recurrent state, and the generic decode path's numerics are followed.

Per decode step the GPU runs 5 kernels per layer plus one for the head:
  full attention : qkv GEMV (+input RMSNorm) -> attention (q/k norm, RoPE,
                   KV write, split-K, gate) -> o_proj GEMV (+residual)
  GatedDeltaNet  : in_proj GEMV x4 (+input RMSNorm) -> GDN step (conv, gates,
                   l2norm, delta rule, gated norm) -> out_proj GEMV (+residual)
  both           : gate/up GEMV (+post-attn RMSNorm, SiLU*up) -> down GEMV
                   (+residual)
  head           : lm_head GEMV (+final RMSNorm) -> greedy argmax -> token,
                   position += 1, next token's embedding row.
Token, position and hidden state stay on the device, so one step is a
replayable HIP graph with no host round trip.
"""

import torch

from . import abi
from . import ops


def rope_tables(max_pos, rotary_dim, theta, device="cpu"):
    """fp32 cos/sin [max_pos, rotary_dim] of the partial rotary embedding, built
    in fp32 on `device` the way main.py:527-533 builds it (inv_freq over the
    rotary dim, freqs = outer(pos, inv_freq), emb = cat(f, f))."""
    inv = 1.0 / (theta ** (torch.arange(0, rotary_dim, 2, device=device).float() / rotary_dim))
    pos = torch.arange(max_pos, device=device).float()
    f = torch.outer(pos, inv)
    emb = torch.cat([f, f], dim=-1)
    return emb.cos().contiguous(), emb.sin().contiguous()


# Prompts of at least this many tokens run the GatedDeltaNet layers in the
# chunked (WY) form on the matrix cores (qh_gdn_chunk); shorter ones use the
# recurrent scan.  At the 4B shape the chunked form measured 38 us against
# 50 us per layer at 128 tokens and 32 us against 31 us at 64.
GDN_CHUNK_MIN_TOKENS = 96


def default_attn_splits(max_seq):
    """Position splits of the decode attention: 64 for a 4096-position cache.
    A split spans one 32-position tile up to 2048 positions, so short contexts
    run the same active splits whatever the count; at context 4096, 64 splits
    (256 workgroups, 2 tiles each) measured 21.4 us against 22.8 us with 32."""
    return max(1, min(64, max_seq // 64))


class Qwen35FP8Engine:
    def __init__(self, weights, max_seq_len=4096, attn_splits=None, device="cuda",
                 batch_prefill=True, split_gdn=True):
        if not torch.cuda.is_available():
            raise RuntimeError("Qwen35FP8Engine needs a GPU (there is no CPU fallback)")
        self.lib = abi.load()
        self.cfg = cfg = weights.cfg
        self.w = weights if weights.embed.is_cuda else weights.to(device)
        self.device = torch.device(device)
        self.max_seq_len = max_seq_len
        self.eps = cfg.rms_norm_eps
        dev = self.device
        bf = dict(dtype=torch.bfloat16, device=dev)
        H, I, V = cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size
        self.h = torch.zeros(H, **bf)
        self.h2 = torch.zeros(H, **bf)
        self.q_all = torch.zeros(cfg.q_proj_rows, **bf)
        self.k_new = torch.zeros(cfg.kv_rows, **bf)
        self.v_new = torch.zeros(cfg.kv_rows, **bf)
        self.mixed = torch.zeros(cfg.conv_dim, **bf)
        self.z = torch.zeros(cfg.value_dim, **bf)
        self.a = torch.zeros(cfg.linear_num_value_heads, **bf)
        self.b = torch.zeros(cfg.linear_num_value_heads, **bf)
        self.mix_out = torch.zeros(max(cfg.attn_out_dim, cfg.value_dim), **bf)
        self.core = torch.zeros(cfg.value_dim, dtype=torch.float32, device=dev)
        self.m = torch.zeros(I, **bf)
        self.logits = torch.zeros(V, **bf)
        self.tok = torch.zeros(1, 1, dtype=torch.int64, device=dev)
        self.tok_hist = torch.zeros(max_seq_len, dtype=torch.int64, device=dev)
        self.pos = torch.zeros(1, dtype=torch.int32, device=dev)
        self._host_pos = 0       # host mirror of pos (bounds the steps the host enqueues)
        self.lm_scratch = torch.zeros(int(self.lib.qh_lm_head_scratch_bytes(V)), dtype=torch.uint8,
                                      device=dev)
        self.lm_counter = torch.zeros(1, dtype=torch.int32, device=dev)
        # nucleus sampling (off: greedy argmax, the benchmark path)
        self.sampling = None
        self.sample_ws = torch.zeros(int(self.lib.qh_sample_workspace_size(V)), dtype=torch.uint8,
                                     device=dev)
        self.sample_ctr = torch.zeros(1, dtype=torch.int64, device=dev)
        self.gen_lo = torch.zeros(1, dtype=torch.int32, device=dev)
        self.sample_info = torch.zeros(16, dtype=torch.int64, device=dev)
        self.attn_splits = attn_splits or default_attn_splits(max_seq_len)
        nbytes = int(self.lib.qh_attn_scratch_bytes(cfg.num_key_value_heads, self.attn_splits,
                                                    cfg.head_dim))
        self.attn_scratch = torch.zeros(max(nbytes, 4), dtype=torch.uint8, device=dev)
        self.attn_counters = torch.zeros(cfg.num_key_value_heads, dtype=torch.int32, device=dev)
        self.gdn_counters = torch.zeros(cfg.linear_num_value_heads, dtype=torch.int32, device=dev)
        self.rope_cos, self.rope_sin = rope_tables(max_seq_len, cfg.rotary_dim, cfg.rope_theta,
                                                   device=dev)
        self.k_cache, self.v_cache, self.conv_ring, self.state = [], [], [], []
        for i in range(cfg.num_hidden_layers):
            if cfg.is_full(i):
                shape = (cfg.num_key_value_heads, max_seq_len, cfg.head_dim)
                self.k_cache.append(torch.zeros(shape, **bf))
                self.v_cache.append(torch.zeros(shape, **bf))
                self.conv_ring.append(None)
                self.state.append(None)
            else:
                self.k_cache.append(None)
                self.v_cache.append(None)
                self.conv_ring.append(torch.zeros(cfg.conv_dim, cfg.linear_conv_kernel_dim, **bf))
                self.state.append(torch.zeros(cfg.linear_num_value_heads, cfg.linear_key_head_dim,
                                              cfg.linear_value_head_dim, dtype=torch.float32,
                                              device=dev))
        self.graph = None
        self.prompt_buf = None
        self.batch_prefill = batch_prefill
        self._pf = None          # prefill buffers, sized for the longest prompt seen
        # GatedDeltaNet decode split in two launches' worth of work: the step up
        # to the bf16 core (qh_gdn_decode_core, one wave per head and 8 value
        # columns), then the gated RMSNorm as the output projection's prologue
        # (qh_gemv_e4m3_gated).  Needs head dims 128, Hv % 8 == 0 and the fast
        # GEMV shape for out_proj; other shapes run the fused step.
        self.split_gdn = split_gdn and self._split_gdn_ok()
        self.gdn_core = torch.zeros(cfg.value_dim, **bf)

    # ------------------------------------------------------------------ state
    def _reset_cache(self):
        """Zero GatedDeltaNet conv/recurrent states; position 0 (main.py:851-895);
        the sampler's draw counter back to 0.  KV-cache contents need no
        clearing: every readable slot is rewritten."""
        for r in self.conv_ring:
            if r is not None:
                r.zero_()
        for s in self.state:
            if s is not None:
                s.zero_()
        self.pos.zero_()
        self._host_pos = 0
        self.sample_ctr.zero_()

    # ------------------------------------------------------------- launches
    def _gemv(self, x, segs, norm_w=None, res=None):
        L = self.lib
        args = []
        for i in range(4):
            if i < len(segs):
                (w, s), y = segs[i]
                args += [abi.ptr(w), abi.ptr(s), abi.ptr(y), w.shape[0], ops.scale_mode(w, s)]
            else:
                args += [None, None, None, 0, 0]
        abi.check(L.qh_gemv_e4m3(abi.ptr(x), None, abi.ptr(norm_w), self.eps, x.numel(),
                                 abi.ptr(res), None, len(segs), *args, 0, abi.stream_handle()),
                  "gemv")

    def _in_segs(self, i):
        """Input projection of layer i: ((w, s), out) segments sharing the
        normalised hidden state."""
        ly = self.w.layers[i]
        if self.cfg.is_full(i):
            return [(ly["q_proj"], self.q_all), (ly["k_proj"], self.k_new),
                    (ly["v_proj"], self.v_new)]
        return [(ly["in_proj_qkv"], self.mixed), (ly["in_proj_z"], self.z),
                (ly["in_proj_a"], self.a), (ly["in_proj_b"], self.b)]

    def _out_proj(self, i):
        ly = self.w.layers[i]
        if self.cfg.is_full(i):
            return self.mix_out[:self.cfg.attn_out_dim], ly["o_proj"]
        return self.mix_out[:self.cfg.value_dim], ly["out_proj"]

    def _split_gdn_ok(self):
        cfg = self.cfg
        if (cfg.linear_key_head_dim, cfg.linear_value_head_dim) != (128, 128) \
                or cfg.linear_num_value_heads % 8 != 0 or cfg.value_dim % 512 != 0:
            return False
        for i in range(cfg.num_hidden_layers):
            if cfg.is_full(i):
                continue
            w, s = self.w.layers[i]["out_proj"]
            if ops.scale_mode(w, s) != w.shape[1] // 128:
                return False
        return True

    def _mixer(self, i):
        cfg, L, ly = self.cfg, self.lib, self.w.layers[i]
        st = abi.stream_handle()
        if cfg.is_full(i):
            D = cfg.head_dim
            gate = self.q_all[D:]
            abi.check(L.qh_attn_decode(
                abi.ptr(self.q_all), 2 * D, abi.ptr(gate), 2 * D, abi.ptr(self.k_new),
                abi.ptr(self.v_new), abi.ptr(ly["q_norm"]), abi.ptr(ly["k_norm"]),
                abi.ptr(self.rope_cos), abi.ptr(self.rope_sin), abi.ptr(self.k_cache[i]),
                abi.ptr(self.v_cache[i]), self.max_seq_len, D, cfg.rotary_dim,
                cfg.num_attention_heads, cfg.num_key_value_heads, abi.ptr(self.pos), 0,
                self.attn_splits, abi.ptr(self.attn_scratch), abi.ptr(self.attn_counters),
                abi.ptr(self.mix_out), self.eps, st), "attn_decode")
        elif self.split_gdn:
            abi.check(L.qh_gdn_decode_core(
                abi.ptr(self.mixed), abi.ptr(self.a), abi.ptr(self.b), abi.ptr(self.conv_ring[i]),
                abi.ptr(ly["conv1d_w"]), abi.ptr(ly["A_log"]), abi.ptr(ly["dt_bias"]),
                abi.ptr(self.state[i]), abi.ptr(self.gdn_core), abi.ptr(self.pos), 0,
                cfg.linear_num_key_heads, cfg.linear_num_value_heads, cfg.linear_key_head_dim,
                cfg.linear_value_head_dim, st), "gdn_decode_core")
        else:
            abi.check(L.qh_gdn_decode(
                abi.ptr(self.mixed), abi.ptr(self.a), abi.ptr(self.b), abi.ptr(self.z),
                abi.ptr(self.conv_ring[i]), abi.ptr(ly["conv1d_w"]), abi.ptr(ly["A_log"]),
                abi.ptr(ly["dt_bias"]), abi.ptr(ly["norm_w"]), abi.ptr(self.state[i]),
                abi.ptr(self.core), abi.ptr(self.mix_out), abi.ptr(self.gdn_counters),
                abi.ptr(self.pos), 0, cfg.linear_num_key_heads, cfg.linear_num_value_heads,
                cfg.linear_key_head_dim, cfg.linear_value_head_dim, self.eps, st), "gdn_decode")

    def _post(self, i):
        """Output projection + residual, gate/up, down + residual (separate launches)."""
        cfg, L, ly = self.cfg, self.lib, self.w.layers[i]
        st = abi.stream_handle()
        x, wo = self._out_proj(i)
        if self.split_gdn and not cfg.is_full(i):
            w, s = wo
            abi.check(L.qh_gemv_e4m3_gated(
                abi.ptr(self.gdn_core), abi.ptr(self.z), abi.ptr(ly["norm_w"]),
                cfg.linear_value_head_dim, self.eps, cfg.value_dim, abi.ptr(self.h), abi.ptr(w),
                abi.ptr(s), abi.ptr(self.h2), w.shape[0], ops.scale_mode(w, s),
                int(s.dtype == torch.bfloat16), st), "gemv_gated")
        else:
            self._gemv(x, [(wo, self.h2)], res=self.h)
        wg, sg = ly["gate_proj"]
        wu, su = ly["up_proj"]
        abi.check(L.qh_mlp_gate_up(abi.ptr(self.h2), None, abi.ptr(ly["post_attention_layernorm"]),
                                   self.eps, cfg.hidden_size, abi.ptr(wg), abi.ptr(sg), abi.ptr(wu),
                                   abi.ptr(su), wg.shape[0], ops.scale_mode(wg, sg),
                                   abi.ptr(self.m), None, None, 0, st), "mlp_gate_up")
        self._gemv(self.m, [(ly["down_proj"], self.h)], res=self.h2)

    def _head(self, next_embed=True):
        cfg, L = self.cfg, self.lib
        abi.check(L.qh_lm_head_argmax(
            abi.ptr(self.h), abi.ptr(self.w.norm_f), self.eps, cfg.hidden_size,
            abi.ptr(self.w.lm_head), cfg.vocab_size, abi.ptr(self.logits),
            abi.ptr(self.lm_scratch), abi.ptr(self.lm_counter), abi.ptr(self.tok),
            abi.ptr(self.tok_hist), self.max_seq_len, abi.ptr(self.pos),
            abi.ptr(self.w.embed) if next_embed else None,
            abi.ptr(self.h) if next_embed else None, abi.stream_handle()), "lm_head_argmax")

    def set_sampling(self, temperature=None, top_p=0.9, rep_penalty=1.0, window=50, seed=0):
        """Sample instead of taking the argmax, with the reference's top_p_sample
        semantics (main.py:49-87; temperature / top-p / repetition penalty over
        the last `window` generated tokens, main.py:1720-1731).  temperature=None
        restores greedy decoding.  A captured graph is dropped: capture again."""
        if temperature is None:
            self.sampling = None
        else:
            if not 0 <= window <= 64:
                raise ValueError("window must be in [0, 64]")
            self.sampling = dict(temperature=float(temperature), top_p=float(top_p),
                                 rep_penalty=float(rep_penalty), window=int(window), seed=int(seed))
        self.graph = None

    def _sample(self):
        """Replace the argmax the head just wrote (token, history slot pos - 1,
        next embedding) by a draw from the nucleus of the same logits."""
        sp = self.sampling
        if sp is None:
            return
        cfg = self.cfg
        abi.check(self.lib.qh_sample_top_p(
            abi.ptr(self.logits), cfg.vocab_size, sp["temperature"], sp["top_p"], sp["rep_penalty"],
            abi.ptr(self.tok_hist), self.max_seq_len, abi.ptr(self.pos), 0, -1,
            abi.ptr(self.gen_lo), sp["window"],
            sp["seed"], abi.ptr(self.sample_ctr), abi.ptr(self.sample_ws), abi.ptr(self.tok),
            abi.ptr(self.w.embed), abi.ptr(self.h), cfg.hidden_size, abi.ptr(self.sample_info),
            abi.stream_handle()), "sample_top_p")

    def _pre(self, i):
        self._gemv(self.h, self._in_segs(i), norm_w=self.w.layers[i]["input_layernorm"])

    def decode_step_launches(self):
        """Enqueue one decode step on the current stream: h holds the input
        token's embedding, pos its position; afterwards logits/tok hold the
        result, h the next token's embedding and pos = pos + 1."""
        n = self.cfg.num_hidden_layers
        self._pre(0)
        for i in range(n):
            self._mixer(i)
            self._post(i)
            if i + 1 < n:
                self._pre(i + 1)
        self._head()
        self._sample()

    # ------------------------------------------------------------ graphs
    def capture(self):
        """Capture one decode step as a HIP graph (replayed by `step`).

        Runs one eager step first (loads every kernel before capture), so the
        recurrent state is reset afterwards: call before prefill."""
        self.decode_step_launches()
        torch.cuda.synchronize()
        self._reset_cache()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.decode_step_launches()
        torch.cuda.synchronize()
        self._reset_cache()
        self.graph = g
        return g

    def _advance(self, n):
        """Host-side mirror of the device position: a decode step consumes the
        token at position pos (KV slot and history entry pos) and leaves
        pos + 1, so n more steps need pos + n <= max_seq_len."""
        if self._host_pos + n > self.max_seq_len:
            raise ValueError(f"{n} decode step(s) from position {self._host_pos} exceed "
                             f"max_seq_len={self.max_seq_len}")
        self._host_pos += n

    def step(self):
        """One greedy decode step from the device-resident token/position."""
        self._advance(1)
        if self.graph is not None:
            self.graph.replay()
        else:
            self.decode_step_launches()

    # ------------------------------------------------------ reference API
    @torch.inference_mode()
    def forward(self, input_ids, past_len=0, logits_to_keep=1):
        """bf16 logits [k, vocab] of the last k = min(logits_to_keep, s) input
        positions, all s for logits_to_keep=0 (main.py:1569-1604).

        past_len == 0 starts a new sequence: the recurrent state, conv ring and
        position are cleared first (the reference ignores the stored recurrent
        state there, main.py:1130-1131, and its callers reset the caches before
        every prompt, main.py:1617/1711).  s > 1 runs the batch prefill at any
        past_len (main.py:1550-1566); s == 1 is one decode step."""
        if isinstance(input_ids, list):
            input_ids = torch.tensor([input_ids], dtype=torch.long, device=self.device)
        ids = input_ids.reshape(-1).to(self.device, torch.int64)
        s = ids.numel()
        if s < 1:
            raise ValueError("forward needs at least one input id")
        if past_len < 0 or past_len + s > self.max_seq_len:
            raise ValueError(f"Sequence range [{past_len}, {past_len + s}) exceeds "
                             f"max_seq_len={self.max_seq_len}")
        if logits_to_keep < 0:
            raise ValueError("logits_to_keep must be non-negative")
        keep = s if logits_to_keep == 0 else min(logits_to_keep, s)
        if past_len == 0:
            self._reset_cache()
        # the sampler's repetition window starts at the first generated token
        self.gen_lo.fill_(past_len + s - 1)
        if s > 1 and self.batch_prefill:
            return self.prefill_batch(ids, past_len, keep)
        st = abi.stream_handle()
        out = None
        if keep > 1:
            out = torch.empty(keep, self.cfg.vocab_size, dtype=torch.bfloat16, device=self.device)
        self.pos.fill_(past_len)
        self._host_pos = past_len
        for t in range(s):
            abi.check(self.lib.qh_embed(abi.ptr(self.w.embed), abi.ptr(ids[t:t + 1]),
                                        abi.ptr(self.h), 1, self.cfg.hidden_size,
                                        self.cfg.vocab_size, st), "embed")
            self.step()
            if out is not None and t >= s - keep:
                out[t - (s - keep)].copy_(self.logits)
        return out if out is not None else self.logits.view(1, -1)

    def prefill(self, ids):
        """Run the prompt; afterwards tok holds the greedy next token, h its
        embedding and pos = len(ids)."""
        self.forward(ids, past_len=0)

    # --------------------------------------------------------- batch prefill
    def _prefill_buffers(self, M):
        if self._pf is not None and self._pf["M"] >= M:
            return self._pf
        cfg, dev = self.cfg, self.device
        bf = dict(dtype=torch.bfloat16, device=dev)
        H, I = cfg.hidden_size, cfg.intermediate_size
        kmax = max(H, I, cfg.attn_out_dim, cfg.value_dim)
        ws = int(self.lib.qh_gemm_workspace_size(M, kmax))
        self._pf = {
            "M": M, "h": torch.empty(M, H, **bf), "hn": torch.empty(M, H, **bf),
            "o": torch.empty(M, H, **bf), "q_all": torch.empty(M, cfg.q_proj_rows, **bf),
            "k": torch.empty(M, cfg.kv_rows, **bf), "v": torch.empty(M, cfg.kv_rows, **bf),
            "q32": torch.empty(M, cfg.num_attention_heads * cfg.head_dim, dtype=torch.float32,
                               device=dev),
            "att": torch.empty(M, cfg.attn_out_dim, **bf),
            "mixed": torch.empty(M, cfg.conv_dim, **bf), "y": torch.empty(M, cfg.conv_dim, **bf),
            "z": torch.empty(M, cfg.value_dim, **bf),
            "a": torch.empty(M, cfg.linear_num_value_heads, **bf),
            "b": torch.empty(M, cfg.linear_num_value_heads, **bf),
            "qn": torch.empty(M, cfg.key_dim, **bf), "kn": torch.empty(M, cfg.key_dim, **bf),
            "g": torch.empty(M, cfg.linear_num_value_heads, dtype=torch.float32, device=dev),
            "beta": torch.empty(M, cfg.linear_num_value_heads, **bf),
            "gated": torch.empty(M, cfg.value_dim, **bf),
            "gu_g": torch.empty(M, I, **bf), "gu_u": torch.empty(M, I, **bf),
            "m": torch.empty(M, I, **bf), "ids": torch.empty(M, dtype=torch.int64, device=dev),
            "ws": torch.empty(max(ws, 16), dtype=torch.uint8, device=dev),
            "gdn_ws": torch.empty(max(int(self.lib.qh_gdn_chunk_workspace_size(
                M, cfg.linear_num_value_heads)), 16), dtype=torch.uint8, device=dev),
        }
        return self._pf

    def _gemm_add_norm(self, x, ws_pair, o, M, ws, h, norm_w, hn):
        """Output projection, residual add and the (1+w) RMSNorm that follows
        (norm_w None: the add only) in qh_gemm_e4m3_add_rmsnorm: h += x W^T
        in bf16, hn = RMSNorm(h); o is scratch."""
        w, s = ws_pair
        abi.check(self.lib.qh_gemm_e4m3_add_rmsnorm(
            abi.ptr(x), abi.ptr(w), abi.ptr(s), abi.ptr(o), M, w.shape[0], w.shape[1],
            ops.scale_mode(w, s), int(s.dtype == torch.bfloat16), abi.ptr(h),
            abi.ptr(norm_w) if norm_w is not None else None, abi.ptr(hn), self.eps, abi.ptr(ws),
            ws.numel(), abi.stream_handle()), "gemm_add_rmsnorm")

    def _gemm_group(self, x, segs, M, ws):
        """Projections [((w, s), y), ...] of the same activation x in one
        qh_gemm_e4m3_grouped launch (1 to 4 segments, one activation split)."""
        args = []
        for i in range(4):
            if i < len(segs):
                (w, s), y = segs[i]
                args += [abi.ptr(w), abi.ptr(s), abi.ptr(y), w.shape[0], ops.scale_mode(w, s)]
            else:
                args += [None, None, None, 0, 0]
        w0, s0 = segs[0][0]
        abi.check(self.lib.qh_gemm_e4m3_grouped(abi.ptr(x), M, w0.shape[1], len(segs), *args,
                                                int(s0.dtype == torch.bfloat16), abi.ptr(ws),
                                                ws.numel(), abi.stream_handle()), "gemm_grouped")

    def prefill_batch(self, ids, past=0, keep=1, trace=None):
        """The reference's s > 1 prefill (main.py:1550-1566) of M tokens at
        positions past .. past + M - 1: every projection as an FP8 GEMM over
        the M tokens, batch attention / GatedDeltaNet kernels continuing from
        the stored KV cache, conv ring and recurrent state (cleared first when
        past == 0), then the lm_head + greedy argmax of the last token.
        Afterwards tok holds the next token, h its embedding and pos = past + M.
        Returns the bf16 logits of the last `keep` tokens [keep, vocab].
        With a list `trace`, the last token's hidden state after each layer is
        appended to it (a host copy per layer: diagnostics only)."""
        cfg, L = self.cfg, self.lib
        ids = ids.reshape(-1).to(self.device, torch.int64)
        M = ids.numel()
        if M < 1 or past < 0 or past + M > self.max_seq_len:
            raise ValueError(f"tokens [{past}, {past + M}) do not fit max_seq_len={self.max_seq_len}")
        if not 1 <= keep <= M:
            raise ValueError(f"keep={keep} outside [1, {M}]")
        B = self._prefill_buffers(M)
        st = abi.stream_handle()
        H, I, eps = cfg.hidden_size, cfg.intermediate_size, self.eps
        if past == 0:
            self._reset_cache()
        h, hn, o, ws = B["h"][:M], B["hn"][:M], B["o"][:M], B["ws"]
        B["ids"][:M].copy_(ids)
        abi.check(L.qh_embed(abi.ptr(self.w.embed), abi.ptr(B["ids"]), abi.ptr(h), M, H,
                             cfg.vocab_size, st), "embed")
        # Each output projection is fused with the residual add and the (1+w)
        # RMSNorm that follow it (qh_gemm_e4m3_add_rmsnorm); layer 0's input
        # norm stands alone and the last layer's final add has no norm after
        # it (lm_head applies norm_f).
        abi.check(L.qh_rmsnorm(abi.ptr(h), abi.ptr(self.w.layers[0]["input_layernorm"]), abi.ptr(hn),
                               M, H, eps, st), "rmsnorm")
        for i in range(cfg.num_hidden_layers):
            ly = self.w.layers[i]
            if cfg.is_full(i):
                D, Hq, Hkv = cfg.head_dim, cfg.num_attention_heads, cfg.num_key_value_heads
                q_all, k, v = B["q_all"][:M], B["k"][:M], B["v"][:M]
                self._gemm_group(hn, [(ly["q_proj"], q_all), (ly["k_proj"], k),
                                      (ly["v_proj"], v)], M, ws)
                abi.check(L.qh_attn_prep(abi.ptr(q_all), abi.ptr(k), abi.ptr(v),
                                         abi.ptr(ly["q_norm"]), abi.ptr(ly["k_norm"]),
                                         abi.ptr(self.rope_cos), abi.ptr(self.rope_sin),
                                         abi.ptr(B["q32"]), abi.ptr(self.k_cache[i]),
                                         abi.ptr(self.v_cache[i]), M, Hq, Hkv, D, cfg.rotary_dim,
                                         past, self.max_seq_len, eps, st), "attn_prep")
                abi.check(L.qh_attn_prefill(abi.ptr(B["q32"]), abi.ptr(q_all[:, D:]), Hq * 2 * D,
                                            2 * D, abi.ptr(self.k_cache[i]),
                                            abi.ptr(self.v_cache[i]), abi.ptr(B["att"]), M, Hq, Hkv,
                                            D, past, self.max_seq_len, st), "attn_prefill")
                self._gemm_add_norm(B["att"][:M], ly["o_proj"], o, M, ws, h, ly["post_attention_layernorm"], hn)
            else:
                Hk, Hv = cfg.linear_num_key_heads, cfg.linear_num_value_heads
                dk, dv = cfg.linear_key_head_dim, cfg.linear_value_head_dim
                self._gemm_group(hn, [(ly["in_proj_qkv"], B["mixed"][:M]), (ly["in_proj_z"], B["z"][:M]),
                                      (ly["in_proj_b"], B["b"][:M]), (ly["in_proj_a"], B["a"][:M])],
                                 M, ws)
                abi.check(L.qh_gdn_prep(abi.ptr(B["mixed"]), abi.ptr(self.conv_ring[i]),
                                        abi.ptr(ly["conv1d_w"]), abi.ptr(B["a"]), abi.ptr(B["b"]),
                                        abi.ptr(ly["A_log"]), abi.ptr(ly["dt_bias"]),
                                        abi.ptr(B["y"]), abi.ptr(B["qn"]), abi.ptr(B["kn"]),
                                        abi.ptr(B["g"]), abi.ptr(B["beta"]), M, Hk, Hv, dk, dv,
                                        past, st), "gdn_prep")
                scan_args = (abi.ptr(B["qn"]), abi.ptr(B["kn"]), abi.ptr(B["y"]), abi.ptr(B["g"]),
                             abi.ptr(B["beta"]), abi.ptr(B["z"]), abi.ptr(ly["norm_w"]),
                             abi.ptr(self.state[i]), abi.ptr(B["gated"]), M, Hk, Hv, dk, dv, 1e-6)
                if M >= GDN_CHUNK_MIN_TOKENS:
                    gws = B["gdn_ws"]
                    abi.check(L.qh_gdn_chunk(*scan_args, abi.ptr(gws), gws.numel(), st), "gdn_chunk")
                else:
                    abi.check(L.qh_gdn_scan(*scan_args, st), "gdn_scan")
                self._gemm_add_norm(B["gated"][:M], ly["out_proj"], o, M, ws, h,
                                    ly["post_attention_layernorm"], hn)
            self._gemm_group(hn, [(ly["gate_proj"], B["gu_g"][:M]), (ly["up_proj"], B["gu_u"][:M])],
                             M, ws)
            abi.check(L.qh_silu_mul(abi.ptr(B["gu_g"]), abi.ptr(B["gu_u"]), abi.ptr(B["m"]), M * I,
                                    st), "silu_mul")
            nxt = self.w.layers[i + 1]["input_layernorm"] if i + 1 < cfg.num_hidden_layers else None
            self._gemm_add_norm(B["m"][:M], ly["down_proj"], o, M, ws, h, nxt, hn)
            if trace is not None:
                trace.append(h[M - 1].float().cpu())
        out = None
        if keep > 1:
            # every kept position but the last: logits only (no token, position
            # or history side effects)
            out = torch.empty(keep, cfg.vocab_size, dtype=torch.bfloat16, device=self.device)
            for j in range(keep - 1):
                r = M - keep + j
                abi.check(L.qh_lm_head_argmax(
                    abi.ptr(h[r]), abi.ptr(self.w.norm_f), eps, H, abi.ptr(self.w.lm_head),
                    cfg.vocab_size, abi.ptr(out[j]), abi.ptr(self.lm_scratch),
                    abi.ptr(self.lm_counter), abi.ptr(self.tok), None, 0, None, None, None, st),
                    "lm_head_argmax")
        self.pos.fill_(past + M - 1)
        self._host_pos = past + M
        abi.check(L.qh_lm_head_argmax(
            abi.ptr(h[M - 1]), abi.ptr(self.w.norm_f), eps, H, abi.ptr(self.w.lm_head),
            cfg.vocab_size, abi.ptr(self.logits), abi.ptr(self.lm_scratch),
            abi.ptr(self.lm_counter), abi.ptr(self.tok), abi.ptr(self.tok_hist), self.max_seq_len,
            abi.ptr(self.pos), abi.ptr(self.w.embed), abi.ptr(self.h), st), "lm_head_argmax")
        self._sample()
        if out is not None:
            out[keep - 1].copy_(self.logits)
            return out
        return self.logits.view(1, -1)

    @torch.inference_mode()
    def decode_trace(self, tok, pos):
        """One eager decode step of token `tok` at position `pos` that also
        returns the hidden state after every layer (host copies; diagnostics
        for per-layer parity against the oracle).  Leaves the engine as
        forward([tok], pos) does; returns (per-layer hidden states, logits)."""
        if pos < 0 or pos >= self.max_seq_len:
            raise ValueError(f"position {pos} outside [0, {self.max_seq_len})")
        if pos == 0:
            self._reset_cache()
        ids = torch.tensor([tok], dtype=torch.int64, device=self.device)
        st = abi.stream_handle()
        abi.check(self.lib.qh_embed(abi.ptr(self.w.embed), abi.ptr(ids), abi.ptr(self.h), 1,
                                    self.cfg.hidden_size, self.cfg.vocab_size, st), "embed")
        self.pos.fill_(pos)
        self._host_pos = pos
        self._advance(1)
        n = self.cfg.num_hidden_layers
        hs = []
        self._pre(0)
        for i in range(n):
            self._mixer(i)
            self._post(i)
            hs.append(self.h.float().cpu())
            if i + 1 < n:
                self._pre(i + 1)
        self._head()
        self._sample()
        return hs, self.logits.float().cpu()

    def generate(self, n_steps):
        """n decode steps (greedy, or sampled after set_sampling) from the
        current device state (no host sync)."""
        if self._host_pos + n_steps > self.max_seq_len:
            raise ValueError(f"{n_steps} decode steps from position {self._host_pos} exceed "
                             f"max_seq_len={self.max_seq_len}")
        for _ in range(n_steps):
            self.step()

    def tokens(self, start, stop):
        """Tokens chosen at positions [start, stop) (device tensor):
        tokens(t, t+1) is the token predicted after consuming position t."""
        return self.tok_hist[start:stop]
