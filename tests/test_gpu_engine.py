"""Whole-model decode parity of the engine against the CPU oracle (MI355X)."""
import pytest
import torch

from oracle import qwen35_oracle as orc
from qwen35_amd import engine as eng_mod
from qwen35_amd.config import tiny
from qwen35_amd.synth import make_prompt, make_weights

from _util import cos_sim

pytestmark = pytest.mark.gpu


def _run(cfg, n_prompt, n_steps, graph):
    w = make_weights(cfg, seed=0)
    prompt = make_prompt(cfg, n=n_prompt, seed=1)
    # the prompt runs through the decode path here (sequential prefill), so
    # that every position is checked against the oracle's decode path
    eng = eng_mod.Qwen35FP8Engine(w, max_seq_len=128, batch_prefill=False)
    if graph:
        eng.capture()
    eng._reset_cache()
    eng.prefill(prompt.view(1, -1).cuda())
    first_logits = eng.logits.float().cpu().clone()
    eng.generate(n_steps - 1)
    torch.cuda.synchronize()
    toks = eng.tokens(n_prompt - 1, n_prompt - 1 + n_steps).cpu().tolist()
    return w, prompt, toks, first_logits, eng


# tiny(): 4 GatedDeltaNet value heads, the fused decode step; lv_heads=8: the
# split step (qh_gdn_decode_core + the gated out_proj prologue, Hv % 8 == 0).
@pytest.mark.parametrize("graph", [False, True])
@pytest.mark.parametrize("lk,lv", [(2, 4), (4, 8)])
def test_tiny_model_greedy_tokens_match_oracle(graph, lk, lv):
    cfg = tiny(num_layers=4, lk_heads=lk, lv_heads=lv)
    n_prompt, n_steps = 6, 12
    w, prompt, toks, first_logits, eng = _run(cfg, n_prompt, n_steps, graph)
    assert eng.split_gdn == (lv % 8 == 0)
    ref = orc.OracleModel(w, max_seq_len=128, prefill="sequential")
    rl = ref.forward(prompt.view(1, -1), 0).view(-1)
    assert cos_sim(first_logits, rl) > 0.9999
    rtoks, margins = [], []
    logits = rl
    pos = n_prompt
    for _ in range(n_steps):
        t = orc.argmax_first(logits)
        rtoks.append(t)
        top = torch.topk(logits, 2).values
        margins.append(float(top[0] - top[1]))
        logits, _ = ref.decode_token(t, pos)
        logits = logits.view(-1)
        pos += 1
    # Greedy tokens must be identical up to the first bf16 near-tie.
    for i, (a, b) in enumerate(zip(toks, rtoks)):
        if a != b:
            assert margins[i] <= 2 ** -6, f"step {i}: token {a} vs oracle {b}, margin {margins[i]}"
            break


def test_graph_replay_equals_eager():
    cfg = tiny(num_layers=4)
    _, _, toks_e, le, _ = _run(cfg, 5, 10, graph=False)
    _, _, toks_g, lg, _ = _run(cfg, 5, 10, graph=True)
    assert toks_e == toks_g
    assert torch.equal(le, lg)


def test_engine_on_loaded_checkpoint_bf16_scales(tmp_path):
    """A checkpoint written in the released layout, loaded like the reference
    loads it (scale_inv rounded to bf16), decodes like the oracle on the same
    loaded weights."""
    from qwen35_amd import loader
    cfg = tiny(num_layers=4)
    loader.save_checkpoint(make_weights(cfg, seed=9), str(tmp_path))
    w = loader.load_checkpoint(str(tmp_path), device="cpu")
    assert w.layers[0]["gate_proj"][1].dtype == torch.bfloat16
    prompt = make_prompt(cfg, n=7, seed=2)
    eng = eng_mod.Qwen35FP8Engine(w, max_seq_len=64)
    logits = eng.forward(prompt.view(1, -1).cuda(), 0).float().cpu().view(-1)
    ref = orc.OracleModel(w, max_seq_len=64, prefill="reference")
    rl = ref.forward(prompt.view(1, -1), 0).view(-1)
    assert cos_sim(logits, rl) > 0.9999
