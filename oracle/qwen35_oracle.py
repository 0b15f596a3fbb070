"""CPU oracle of the reference engine's batch-1 FP8 path.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module, and only as the checker (or as the
timed CPU baseline); the product path never calls it.

It restates, in plain PyTorch on the CPU (fp32 arithmetic, explicit bf16
rounding wherever the reference materialises a bf16 tensor), the reference's
explicit block-dequant path:
  * E4M3FN decode and the 128x128 block dequant (fp8_kernels.cu:15-17,
    main.py:497-501, scale modes main.py:249-251 / fused_kernels.cu:98-107);
  * the generic decode path of main.py (``_decode_step`` main.py:1509-1547)
    with the DLL kernels it calls by default: launch_rmsnorm_ip
    (fused_kernels.cu:521-547), layer_mid_attn (1224-1297),
    launch_delta_rule_decode (623-684), layer_post_o_fp8_mlp (1156-1195);
    torch glue of main.py:981-1162 (gate, conv update, gates, RMSNormGated);
  * the batch prefill path (``_prefill_step`` main.py:1550-1566) with the
    fp32 torch attention of main.py:1034-1056 and the gated delta rule in its
    recurrent form (equal to transformers' chunked form up to fp32 rounding;
    tests pin that against transformers' own function);
  * top_p_sample (main.py:49-87) without the draw: the kept nucleus and its
    probabilities.
Nothing here imports the product package.
"""
import math

import torch
import torch.nn.functional as F

BLOCK = 128

# Arithmetic type of the model path: float32 (the oracle every test compares
# with) or float64 (the exact path: every intermediate in double precision,
# rounded to bf16 only where the reference materialises a bf16 tensor; with
# MATMUL = "fp64" below).  Only the noise-floor fixture generator
# (tests/golden/make_noise_floor.py) sets float64.
ACC = torch.float32


def _a(x):
    """x in the model path's arithmetic type (ACC)."""
    return x.to(ACC)


def bf16(x):
    """Materialise as bf16 (RNE) and come back to the arithmetic type (fp32)."""
    return x.to(torch.bfloat16).to(ACC)


# ---------------------------------------------------------------- A0: E4M3FN
def e4m3_decode(code):
    """OCP E4M3FN: bias 7, no infinities, S.1111.111 = NaN, subnormal m * 2^-9."""
    sign = -1.0 if code & 0x80 else 1.0
    e = (code >> 3) & 0xF
    m = code & 0x7
    if e == 0xF and m == 0x7:
        return float("nan")
    if e == 0:
        return sign * m * 2.0 ** -9
    return sign * (1.0 + m / 8.0) * 2.0 ** (e - 7)


_TABLE = None


def e4m3_table():
    global _TABLE
    if _TABLE is None:
        _TABLE = torch.tensor([e4m3_decode(c) for c in range(256)], dtype=torch.float32)
    return _TABLE


# ------------------------------------------------------- A10 / A1 dequant, GEMV
def quantize_block_fp8(w, block=BLOCK):
    """main.py:833-848 with an fp32 scale: s = max(amax/448, 1e-12) per block,
    q = e4m3fn_RNE(W / s)."""
    w = w.float()
    N, K = w.shape
    nb, kb = math.ceil(N / block), math.ceil(K / block)
    pad = torch.zeros(nb * block, kb * block)
    pad[:N, :K] = w
    blocks = pad.view(nb, block, kb, block)
    s = (blocks.abs().amax(dim=(1, 3)) / 448.0).clamp(min=1e-12)
    q = (blocks / s.view(nb, 1, kb, 1)).to(torch.float8_e4m3fn).reshape(nb * block, kb * block)
    return q[:N, :K].contiguous().view(torch.uint8), s


def scale_code(w_u8, s):
    """The reference's `K_blocks` argument for a scale tensor (main.py:249-251)."""
    kb = s.shape[1] if s.dim() == 2 else 1
    if s.dim() == 2 and s.shape[0] == w_u8.shape[0] and kb > 1:
        return -kb
    return kb


def dequant(w_u8, s, code=None):
    """fp32 W_deq = e4m3(W) * s broadcast per the scale mode."""
    W = e4m3_table()[w_u8.long()]
    N, K = W.shape
    s = s.float()
    code = scale_code(w_u8, s) if code is None else code
    if code > 1:  # [ceil(N/128), K/128] block scales
        full = s.repeat_interleave(BLOCK, 0).repeat_interleave(BLOCK, 1)[:N, :K]
    elif code == 1:  # per output row
        full = s.reshape(-1)[:N].view(N, 1)
    else:  # [N, K/128] per row and K block
        full = s.view(N, -1).repeat_interleave(BLOCK, 1)[:, :K]
    return W * full


# How the weight products accumulate.  "fp32": one fp32 matmul (what every
# test compares with).  "fp64": fp64 accumulation of the same fp32 operands.
# "kblock": fp32 partial sums per 128-wide K block, added block by block in
# fp32 (the order of the reference's block-scaled kernels, fused_kernels.cu:
# 127-145).  Only the noise-floor fixture generator
# (tests/golden/make_noise_floor.py) sets anything but "fp32": three exact
# restatements of the same path that differ only in rounding.
MATMUL = "fp32"


def wmm(x, W):
    """x @ W^T (x [..., K], W [N, K] fp32), accumulated as MATMUL says; fp32."""
    if MATMUL == "fp32":
        return _a(x.float() @ W.t())
    if MATMUL == "fp64":
        xd = x.double()
        parts = [_a(xd @ W[n0:n0 + 8192].double().t()) for n0 in range(0, W.shape[0], 8192)]
        return torch.cat(parts, dim=-1)
    if MATMUL == "kblock":
        x = x.float()
        out = None
        for k0 in range(0, x.shape[-1], BLOCK):
            p = x[..., k0:k0 + BLOCK] @ W[:, k0:k0 + BLOCK].t()
            out = p if out is None else out + p
        return _a(out)
    raise ValueError(f"unknown MATMUL mode {MATMUL!r}")


def linear(x, W):
    """bf16(x @ W^T) with fp32 accumulation (fp8_linear / F.linear output)."""
    return bf16(wmm(x, W))


def gemv_fp64(x, w_u8, s):
    """Brute force in float64 (no bf16 rounding) for pinning."""
    return x.double() @ dequant(w_u8, s).double().t()


# ------------------------------------------------------------ A3 RMSNorm
def rmsnorm(x, w, eps=1e-6):
    """(1+w) RMSNorm, bf16 output (main.py:921-924, fused_kernels.cu:540-546)."""
    x = _a(x)
    r = torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)
    return bf16((x * r) * (1.0 + _a(w)))


# --------------------------------------------------------------- A2 MLP
def mlp_decode(h, o, ln_w, Wg, Wu, Wd, eps=1e-6):
    """layer_post_o_fp8_mlp (fused_kernels.cu:1156-1195): h2 = bf16(h + o);
    SiLU on the fp32 gate/up accumulators (fused_kernels.cu:476)."""
    h2 = bf16(_a(h) + _a(o))
    xn = rmsnorm(h2, ln_w, eps)
    g = wmm(xn, Wg)
    u = wmm(xn, Wu)
    m = bf16(F.silu(g) * u)
    d = linear(m, Wd)
    return bf16(h2 + d), m


def mlp_prefill(xn, Wg, Wu, Wd):
    """mlp_forward with M > 1 (main.py:1203-1217): bf16 gate/up, bf16 SiLU*up."""
    g = linear(xn, Wg)
    u = linear(xn, Wu)
    m = bf16(bf16(F.silu(g)) * u)
    return linear(m, Wd)


# ------------------------------------------------------------ A4 attention
def rope_tables(max_pos, rot, theta):
    """fp32 cos/sin [max_pos, rot], built in fp32 exactly as main.py:527-533:
    inv_freq = 1 / theta^(arange(0, rot, 2) / rot), freqs = outer(pos, inv_freq),
    emb = cat(freqs, freqs)."""
    inv = 1.0 / (theta ** (torch.arange(0, rot, 2).float() / rot))
    f = torch.outer(torch.arange(max_pos).float(), inv)
    emb = torch.cat([f, f], dim=-1)
    return emb.cos().contiguous(), emb.sin().contiguous()


def rope_rows(x, cos_row, sin_row, rot, round_out):
    """Partial RoPE on dims [0, rot) of each row: pairs (c, c + rot/2)
    (fused_kernels.cu:872-903 decode, main.py:964-976 prefill)."""
    half = rot // 2
    x = _a(x)
    x0, x1 = x[..., :half], x[..., half:rot]
    c0, c1 = cos_row[..., :half], cos_row[..., half:rot]
    s0, s1 = sin_row[..., :half], sin_row[..., half:rot]
    r0 = x0 * c0 - x1 * s0
    r1 = x1 * c1 + x0 * s1
    if round_out:
        r0, r1 = bf16(r0), bf16(r1)
    return torch.cat([r0, r1, x[..., rot:]], dim=-1)


def attn_core(q, K, V):
    """softmax(q K^T / sqrt(D)) V in fp32 for one head; q [D] or [s, D]."""
    D = q.shape[-1]
    sc = (_a(q) @ _a(K).t()) * (1.0 / math.sqrt(D))
    return torch.softmax(sc, dim=-1) @ _a(V)


def attn_decode(q_all, k_new, v_new, q_norm, k_norm, cos, sin, k_cache, v_cache, pos, n_heads,
                n_kv, head_dim, rot, eps=1e-6):
    """layer_mid_attn + sigmoid gate (main.py:1001-1059) for one token at `pos`.
    q_all: [n_heads * 2 * D] with per-head [q | gate]; caches [n_kv, max_seq, D]
    (updated in place).  Returns the gated bf16 output [n_heads * D]."""
    D = head_dim
    qa = _a(q_all).view(n_heads, 2 * D)
    q, gate = qa[:, :D], qa[:, D:]
    q = rmsnorm(q, q_norm, eps) if q_norm is not None else q
    k = rmsnorm(_a(k_new).view(n_kv, D), k_norm, eps) if k_norm is not None else _a(k_new).view(n_kv, D)
    q = rope_rows(q, cos[pos], sin[pos], rot, round_out=True)
    k = rope_rows(k, cos[pos], sin[pos], rot, round_out=True)
    k_cache[:, pos] = k
    v_cache[:, pos] = _a(v_new).view(n_kv, D)
    out = torch.empty(n_heads, D, dtype=ACC)
    for h in range(n_heads):
        kv = h * n_kv // n_heads
        out[h] = bf16(attn_core(q[h], k_cache[kv, :pos + 1], v_cache[kv, :pos + 1]))
    return bf16(out * bf16(torch.sigmoid(gate))).reshape(-1)


def attn_only(q, k_cache, v_cache, seq_len, n_heads, n_kv):
    """launch_fused_attn_v2 semantics: no norm, no RoPE, no cache write."""
    D = k_cache.shape[-1]
    q = q.float().view(n_heads, D)
    out = torch.empty(n_heads, D)
    for h in range(n_heads):
        kv = h * n_kv // n_heads
        out[h] = bf16(attn_core(q[h], k_cache[kv, :seq_len], v_cache[kv, :seq_len]))
    return out.reshape(-1)


# ------------------------------------------------------------ A5 GatedDeltaNet
def softplus(x):
    """torch softplus (beta 1, threshold 20)."""
    return F.softplus(x)


def conv_update(x, state, w):
    """transformers causal_conv1d_update (modeling_qwen3_5.py:200-217) for one
    token: window = [state | x], state <- last 4, y = bf16(silu(bf16(conv))).
    x [C], state [C, 4] ordered oldest..newest (updated in place), w [C, 4]."""
    win = torch.cat([_a(state), _a(x).view(-1, 1)], dim=1)
    state.copy_(win[:, 1:])
    y = bf16((_a(w) * win[:, 1:]).sum(dim=1))
    return bf16(F.silu(y))


def linear_gates(a, b, A_log, dt_bias):
    """beta = bf16(sigmoid(b)); g = -exp(A_log) * softplus(a + dt_bias) (main.py:1120-1122)."""
    beta = bf16(torch.sigmoid(_a(b)))
    g = -torch.exp(_a(A_log)) * softplus(_a(a) + _a(dt_bias))
    return g, beta


def delta_rule_step(q, k, v, g, beta, S):
    """launch_delta_rule_decode (fused_kernels.cu:623-684): fp32 l2norm of q and
    k (eps inside the rsqrt of the sum), q scaled by 1/sqrt(dk); S [H, dk, dv]
    updated in place; returns bf16 o [H, dv]."""
    q, k, v = _a(q), _a(k), _a(v)
    dk = q.shape[-1]
    qn = q * torch.rsqrt((q * q).sum(-1, keepdim=True) + 1e-6) * (1.0 / math.sqrt(dk))
    kn = k * torch.rsqrt((k * k).sum(-1, keepdim=True) + 1e-6)
    decay = torch.exp(_a(g)).view(-1, 1, 1)
    Sd = S * decay
    pred = (Sd * kn.unsqueeze(-1)).sum(dim=-2)
    delta = (v - pred) * _a(beta).view(-1, 1)
    S.copy_(Sd + kn.unsqueeze(-1) * delta.unsqueeze(-2))
    return bf16((S * qn.unsqueeze(-1)).sum(dim=-2))


def gated_rmsnorm(core, z, w, eps=1e-6, bf16_steps=True):
    """Per head [H, dv]: main.py:1152-1158 (bf16_steps) or the fused kernel
    fused_kernels.cu:592-618 (fp32 throughout)."""
    c = _a(core)
    r = torch.rsqrt(c.pow(2).mean(-1, keepdim=True) + eps)
    if bf16_steps:
        normed = bf16(bf16(c * r) * _a(w))
        return bf16(normed * bf16(F.silu(_a(z))))
    return bf16(c * r * _a(w) * F.silu(_a(z)))


def l2norm_bf16(x, eps=1e-6):
    """transformers l2norm applied to a bf16 tensor (every op rounds to bf16),
    as torch_chunk_gated_delta_rule(use_qk_l2norm_in_kernel=True) does in prefill."""
    x = bf16(x)
    ss = bf16(bf16(x * x).sum(-1, keepdim=True))
    inv = bf16(torch.rsqrt(bf16(ss + eps)))
    return bf16(x * inv)


def gated_delta_rule_seq(q, k, v, g, beta, S):
    """Recurrent gated delta rule over a sequence (fp32), q/k already
    normalised, q already scaled.  q,k [T, H, dk], v [T, H, dv], g/beta [T, H];
    S [H, dk, dv] updated in place; returns fp32 o [T, H, dv]."""
    T = q.shape[0]
    out = torch.empty(T, q.shape[1], v.shape[-1], dtype=ACC)
    for t in range(T):
        S.mul_(torch.exp(g[t]).view(-1, 1, 1))
        mem = (S * k[t].unsqueeze(-1)).sum(dim=-2)
        delta = (v[t] - mem) * beta[t].view(-1, 1)
        S.add_(k[t].unsqueeze(-1) * delta.unsqueeze(-2))
        out[t] = (S * q[t].unsqueeze(-1)).sum(dim=-2)
    return out


def chunk_gated_delta_rule(q, k, v, g, beta, chunk=64, S0=None):
    """Chunked (WY) gated delta rule, restating the algorithm transformers
    implements in torch_chunk_gated_delta_rule (modeling_qwen3_5.py:249-328):
    within a chunk, the triangular system (I + tril(diag(beta) K K^T * decay))
    is solved by forward substitution; chunks are chained through the state,
    which starts at S0 [H, dk, dv] (the reference's initial_state, main.py:1130,
    passed when past_len > 0) or zero.  Inputs as gated_delta_rule_seq.
    Returns (o [T, H, dv], S [H, dk, dv])."""
    T, H, dk = k.shape
    dv = v.shape[-1]
    pad = (chunk - T % chunk) % chunk
    def P(x):
        return torch.cat([x, torch.zeros(pad, *x.shape[1:])], 0) if pad else x
    q, k, v, g, beta = P(q), P(k), P(v), P(g), P(beta)
    n = (T + pad) // chunk
    S = torch.zeros(H, dk, dv) if S0 is None else S0.clone().float()
    out = torch.zeros(T + pad, H, dv)
    for c in range(n):
        sl = slice(c * chunk, (c + 1) * chunk)
        for h in range(H):
            qc, kc, vc = q[sl, h], k[sl, h], v[sl, h]
            gc = torch.cumsum(g[sl, h], 0)
            bc = beta[sl, h]
            decay = torch.exp(gc.view(-1, 1) - gc.view(1, -1)).tril()
            A = -((kc * bc.view(-1, 1)) @ kc.t() * decay).tril(-1)
            Tm = torch.eye(chunk)
            for i in range(1, chunk):  # forward substitution: Tm = (I - A)^-1 = I + A Tm
                Tm[i, :i] = A[i, :i] @ Tm[:i, :i]
            u = Tm @ (vc * bc.view(-1, 1))
            w = Tm @ (kc * (bc * torch.exp(gc)).view(-1, 1))
            vnew = u - w @ S[h]
            att = (qc @ kc.t() * decay).tril()
            out[sl, h] = (qc * torch.exp(gc).view(-1, 1)) @ S[h] + att @ vnew
            S[h] = S[h] * torch.exp(gc[-1]) + (kc * torch.exp(gc[-1] - gc).view(-1, 1)).t() @ vnew
    return out[:T], S


# ------------------------------------------------------------- A6 lm_head
def argmax_first(x):
    """Index of the first maximum (torch.argmax semantics on ties)."""
    x = x.float().reshape(-1)
    m = x.max()
    return int(torch.nonzero(x == m)[0].item())


def lm_head_argmax(h, norm_f, lm_head, eps=1e-6):
    xn = rmsnorm(h, norm_f, eps)
    logits = linear(xn, lm_head.float())
    return logits, argmax_first(logits)


# ------------------------------------------------- sampling (main.py:49-87)
def _recip32(x):
    """fp32 reciprocal of a Python float: the reference divides a CUDA tensor by
    a Python scalar, which PyTorch's CUDA kernel computes as a multiplication by
    the fp32 reciprocal."""
    return (torch.tensor(1.0, dtype=torch.float32) / torch.tensor(x, dtype=torch.float32)).item()


def sample_scale(logits, temperature, rep_penalty=1.0, recent_ids=None):
    """main.py:54-63 on a bf16 [V] row: y = bf16(x * (1/T)) when T > 0; then,
    for each distinct recent id, bf16(y * rp) if y < 0 else bf16(y * (1/rp)).
    Returns fp32 values of the bf16 tensor."""
    y = logits.float().reshape(-1).clone()
    if temperature > 0:
        y = bf16(y * _recip32(temperature))
    if rep_penalty > 1.0 and recent_ids:
        ids = torch.tensor(sorted({int(i) for i in recent_ids}), dtype=torch.long)
        r = y[ids]
        y[ids] = torch.where(r < 0, bf16(r * rep_penalty), bf16(r * _recip32(rep_penalty)))
    return y


def sample_nucleus(logits, temperature=0.7, top_p=0.9, rep_penalty=1.0, recent_ids=None,
                   topk=2000, logz_b=None, soft_mz=None):
    """The kept prefix of top_p_sample (main.py:64-82), before the draw.

    Tokens sorted by y descending, ties by index (a stable sort);
    p = bf16(exp(bf16(y - bf16(logsumexp(y))))); when the top-min(topk, V)
    mass, rounded to bf16, is below bf16(top_p), the full-vocabulary softmax
    bf16(exp(y - max) / Z) instead; keep the prefix whose running mass, rounded
    to bf16, stays <= bf16(top_p), at least one token.  logz_b and soft_mz =
    (max, Z) override the log-partition and the softmax normaliser (to check a
    cut with the device's fp32 sums).  Returns (ids, probs, fallback)."""
    y = sample_scale(logits, temperature, rep_penalty, recent_ids)
    V = y.numel()
    order = torch.sort(y, descending=True, stable=True).indices
    ys = y[order]
    if logz_b is None:
        logz_b = bf16(torch.logsumexp(y, 0)).item()
    tp = bf16(torch.tensor(float(top_p))).item()
    p = bf16(torch.exp(bf16(ys - logz_b)))
    k = min(topk, V)
    fallback = bf16(p[:k].double().sum().float()).item() < tp
    if fallback:
        M, Z = soft_mz if soft_mz is not None else (y.max().item(), torch.exp(y - y.max()).sum().item())
        p = bf16(torch.exp(ys - M) / Z)
    cum = bf16(torch.cumsum(p.double(), 0).float())
    n = max(1, int((cum <= tp).sum()))  # cum is non-decreasing: the kept set is a prefix
    return order[:n], p[:n], fallback


# ------------------------------------------------------------------ model
class OracleModel:
    """Whole-model restatement of QwenEngineFP8Opt (main.py:326-1604).

    prefill="reference": s > 1 runs the batch prefill path (main.py:1550-1566);
    prefill="sequential": every prompt token goes through the decode path."""

    def __init__(self, weights, max_seq_len=256, prefill="reference"):
        self.w = weights
        self.cfg = cfg = weights.cfg
        self.max_seq_len = max_seq_len
        self.prefill_mode = prefill
        self.eps = cfg.rms_norm_eps
        self.layers = []
        for ly in weights.layers:
            d = {}
            for k, v in ly.items():
                if isinstance(v, tuple):
                    d[k] = dequant(v[0].cpu(), v[1].cpu())
                elif isinstance(v, torch.Tensor):
                    d[k] = v.detach().cpu().float()
                else:
                    d[k] = v
            self.layers.append(d)
        self.embed = weights.embed.cpu().float()
        self.lm_head = weights.lm_head.cpu().float()
        self.norm_f = weights.norm_f.cpu().float()
        self.cos, self.sin = rope_tables(max_seq_len, cfg.rotary_dim, cfg.rope_theta)
        self._reset_cache()

    def _reset_cache(self):
        cfg = self.cfg
        self.k_cache, self.v_cache, self.conv_state, self.rec_state = [], [], [], []
        for i in range(cfg.num_hidden_layers):
            if cfg.is_full(i):
                shp = (cfg.num_key_value_heads, self.max_seq_len, cfg.head_dim)
                self.k_cache.append(torch.zeros(shp, dtype=ACC))
                self.v_cache.append(torch.zeros(shp, dtype=ACC))
                self.conv_state.append(None)
                self.rec_state.append(None)
            else:
                self.k_cache.append(None)
                self.v_cache.append(None)
                self.conv_state.append(torch.zeros(cfg.conv_dim, cfg.linear_conv_kernel_dim, dtype=ACC))
                self.rec_state.append(torch.zeros(cfg.linear_num_value_heads,
                                                  cfg.linear_key_head_dim,
                                                  cfg.linear_value_head_dim, dtype=ACC))

    # ---- decode (s == 1) ---------------------------------------------------
    def _full_decode(self, i, hn, pos):
        cfg, ly = self.cfg, self.layers[i]
        q_all = linear(hn, ly["q_proj"])
        k = linear(hn, ly["k_proj"])
        v = linear(hn, ly["v_proj"])
        att = attn_decode(q_all, k, v, ly["q_norm"], ly["k_norm"], self.cos, self.sin,
                          self.k_cache[i], self.v_cache[i], pos, cfg.num_attention_heads,
                          cfg.num_key_value_heads, cfg.head_dim, cfg.rotary_dim, self.eps)
        return linear(att, ly["o_proj"])

    def _gdn_decode(self, i, hn):
        cfg, ly = self.cfg, self.layers[i]
        mixed = linear(hn, ly["in_proj_qkv"])
        z = linear(hn, ly["in_proj_z"])
        b = linear(hn, ly["in_proj_b"])
        a = linear(hn, ly["in_proj_a"])
        y = conv_update(mixed, self.conv_state[i], ly["conv1d_w"])
        kd, Hk, Hv = cfg.key_dim, cfg.linear_num_key_heads, cfg.linear_num_value_heads
        dk, dv = cfg.linear_key_head_dim, cfg.linear_value_head_dim
        q = y[:kd].view(Hk, dk).repeat_interleave(Hv // Hk, dim=0)
        k = y[kd:2 * kd].view(Hk, dk).repeat_interleave(Hv // Hk, dim=0)
        v = y[2 * kd:].view(Hv, dv)
        g, beta = linear_gates(a, b, ly["A_log"], ly["dt_bias"])
        core = delta_rule_step(q, k, v, g, beta, self.rec_state[i])
        gated = gated_rmsnorm(core, z.view(Hv, dv), ly["norm_w"], 1e-6, bf16_steps=True)
        return linear(gated.reshape(-1), ly["out_proj"])

    def decode_token(self, tok, pos, trace=None):
        """One decode step (main.py:1509-1547); with a list `trace`, the hidden
        state after every layer is appended to it."""
        cfg = self.cfg
        h = _a(self.embed[tok])
        for i in range(cfg.num_hidden_layers):
            ly = self.layers[i]
            hn = rmsnorm(h, ly["input_layernorm"], self.eps)
            o = self._full_decode(i, hn, pos) if cfg.is_full(i) else self._gdn_decode(i, hn)
            h, _ = mlp_decode(h, o, ly["post_attention_layernorm"], ly["gate_proj"],
                              ly["up_proj"], ly["down_proj"], self.eps)
            if trace is not None:
                trace.append(h.clone())
        logits, tok = lm_head_argmax(h, self.norm_f, self.lm_head, self.eps)
        return logits, tok

    # ---- prefill (s > 1) ----------------------------------------------------
    def _full_prefill(self, i, hn, past):
        cfg, ly = self.cfg, self.layers[i]
        s, D, Hq, Hkv = hn.shape[0], cfg.head_dim, cfg.num_attention_heads, cfg.num_key_value_heads
        q_all = linear(hn, ly["q_proj"]).view(s, Hq, 2 * D)
        q, gate = q_all[..., :D], q_all[..., D:].reshape(s, Hq * D)
        k = linear(hn, ly["k_proj"]).view(s, Hkv, D)
        v = linear(hn, ly["v_proj"]).view(s, Hkv, D)
        q = rmsnorm(q, ly["q_norm"], self.eps)
        k = rmsnorm(k, ly["k_norm"], self.eps)
        cos = self.cos[past:past + s].view(s, 1, -1)
        sin = self.sin[past:past + s].view(s, 1, -1)
        q = rope_rows(q, cos, sin, cfg.rotary_dim, round_out=False)   # stays fp32
        k = rope_rows(k, cos, sin, cfg.rotary_dim, round_out=False)
        self.k_cache[i][:, past:past + s] = bf16(k).transpose(0, 1)
        self.v_cache[i][:, past:past + s] = v.transpose(0, 1)
        total = past + s
        out = torch.empty(s, Hq, D, dtype=ACC)
        mask = torch.triu(torch.full((s, total), float("-inf")), diagonal=1 + past)
        for h in range(Hq):
            kv = h * Hkv // Hq
            sc = (q[:, h] @ self.k_cache[i][kv, :total].t()) * (D ** -0.5) + mask
            out[:, h] = bf16(torch.softmax(sc, dim=-1) @ self.v_cache[i][kv, :total])
        out = bf16(out.reshape(s, Hq * D) * bf16(torch.sigmoid(gate)))
        return linear(out, ly["o_proj"])

    def _gdn_prefill(self, i, hn, past=0):
        cfg, ly = self.cfg, self.layers[i]
        s = hn.shape[0]
        mixed = linear(hn, ly["in_proj_qkv"])
        z = linear(hn, ly["in_proj_z"])
        b = linear(hn, ly["in_proj_b"])
        a = linear(hn, ly["in_proj_a"])
        st = self.conv_state[i]
        xt = torch.cat([st, mixed.t()], dim=1)           # [C, 4 + s]
        st.copy_(xt[:, -st.shape[1]:])
        w = ly["conv1d_w"]
        conv = torch.stack([(w * xt[:, j + 1:j + 5]).sum(1) for j in range(s)], dim=0)
        y = bf16(F.silu(bf16(conv)))                     # [s, C]
        kd, Hk, Hv = cfg.key_dim, cfg.linear_num_key_heads, cfg.linear_num_value_heads
        dk, dv = cfg.linear_key_head_dim, cfg.linear_value_head_dim
        r = Hv // Hk
        q = l2norm_bf16(y[:, :kd].reshape(s, Hk, dk).repeat_interleave(r, dim=1))
        k = l2norm_bf16(y[:, kd:2 * kd].reshape(s, Hk, dk).repeat_interleave(r, dim=1))
        v = y[:, 2 * kd:].reshape(s, Hv, dv)
        g, beta = linear_gates(a, b, ly["A_log"], ly["dt_bias"])
        S = self.rec_state[i]
        if past == 0:
            S.zero_()   # initial_state=None at past_len == 0 (main.py:1130-1131)
        o = gated_delta_rule_seq(q * (1.0 / math.sqrt(dk)), k, v, g, beta, S)
        gated = gated_rmsnorm(bf16(o), z.view(s, Hv, dv), ly["norm_w"], 1e-6, bf16_steps=True)
        return linear(gated.reshape(s, -1), ly["out_proj"])

    def prefill(self, ids, past=0, keep=1, trace=None):
        """Batch prefill of tokens at positions past .. past + s - 1
        (main.py:1550-1566); logits [keep, V] of the last `keep` positions and
        the greedy token after the last one.  With a list `trace`, the last
        token's hidden state after every layer is appended to it."""
        cfg = self.cfg
        h = _a(self.embed[ids])
        for i in range(cfg.num_hidden_layers):
            ly = self.layers[i]
            hn = rmsnorm(h, ly["input_layernorm"], self.eps)
            o = (self._full_prefill(i, hn, past) if cfg.is_full(i)
                 else self._gdn_prefill(i, hn, past))
            h = bf16(h + o)
            hn = rmsnorm(h, ly["post_attention_layernorm"], self.eps)
            h = bf16(h + mlp_prefill(hn, ly["gate_proj"], ly["up_proj"], ly["down_proj"]))
            if trace is not None:
                trace.append(h[-1].clone())
        rows = [lm_head_argmax(r, self.norm_f, self.lm_head, self.eps) for r in h[-keep:]]
        return torch.stack([r[0].reshape(-1) for r in rows]), rows[-1][1]

    # ---- API ----------------------------------------------------------------
    def forward(self, input_ids, past_len=0, logits_to_keep=1):
        """Logits [k, V] of the last k = min(logits_to_keep, s) positions (all s
        for 0), main.py:1569-1604.  past_len == 0 starts a new sequence with
        cleared caches, as the reference's callers do (main.py:1617, 1711)."""
        ids = [int(t) for t in torch.as_tensor(input_ids).reshape(-1)]
        s = len(ids)
        if logits_to_keep < 0:
            raise ValueError("logits_to_keep must be non-negative")
        keep = s if logits_to_keep == 0 else min(logits_to_keep, s)
        if past_len == 0:
            self._reset_cache()
        if s == 1 or self.prefill_mode == "sequential":
            rows = []
            for j, t in enumerate(ids):
                logits, _ = self.decode_token(t, past_len + j)
                if j >= s - keep:
                    rows.append(logits.reshape(-1))
            return torch.stack(rows)
        logits, _ = self.prefill(torch.tensor(ids), past_len, keep)
        return logits

    def greedy(self, prompt, n_steps):
        """Prompt, then n greedy steps; returns the n generated tokens and the
        top-2 logit margin of each step."""
        logits = self.forward(prompt, 0)
        pos = len(prompt)
        toks, margins = [], []
        for _ in range(n_steps):
            tok = argmax_first(logits)
            top = torch.topk(logits.view(-1), 2).values
            toks.append(tok)
            margins.append(float(top[0] - top[1]))
            logits, _ = self.decode_token(tok, pos)
            pos += 1
        return toks, margins
