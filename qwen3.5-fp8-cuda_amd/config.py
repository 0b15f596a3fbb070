"""Model shape description (config.json keys of the reference, main.py:335-370).

Only the text decoder of the hybrid Qwen3.5 family is described: GatedDeltaNet
("linear_attention") layers interleaved with gated GQA ("full_attention")
layers, layer i being full attention iff (i + 1) % full_attention_interval == 0.
"""
import dataclasses
import json


@dataclasses.dataclass
class Qwen35Config:
    vocab_size: int = 248320
    hidden_size: int = 2560
    intermediate_size: int = 9216
    num_hidden_layers: int = 32
    num_attention_heads: int = 16
    num_key_value_heads: int = 4
    head_dim: int = 256
    rope_theta: float = 10000000.0
    partial_rotary_factor: float = 0.25
    rms_norm_eps: float = 1e-6
    linear_num_key_heads: int = 16
    linear_num_value_heads: int = 32
    linear_key_head_dim: int = 128
    linear_value_head_dim: int = 128
    linear_conv_kernel_dim: int = 4
    full_attention_interval: int = 4
    layer_types: list = None

    def __post_init__(self):
        if self.layer_types is None:
            self.layer_types = [
                "full_attention" if (i + 1) % self.full_attention_interval == 0
                else "linear_attention"
                for i in range(self.num_hidden_layers)
            ]
        if len(self.layer_types) != self.num_hidden_layers:
            raise ValueError("layer_types must have num_hidden_layers entries")

    # derived sizes -----------------------------------------------------------
    @property
    def rotary_dim(self):
        return int(self.head_dim * self.partial_rotary_factor)

    @property
    def q_proj_rows(self):  # gated q: per head [q (head_dim) | gate (head_dim)]
        return self.num_attention_heads * self.head_dim * 2

    @property
    def kv_rows(self):
        return self.num_key_value_heads * self.head_dim

    @property
    def attn_out_dim(self):
        return self.num_attention_heads * self.head_dim

    @property
    def key_dim(self):
        return self.linear_num_key_heads * self.linear_key_head_dim

    @property
    def value_dim(self):
        return self.linear_num_value_heads * self.linear_value_head_dim

    @property
    def conv_dim(self):
        return 2 * self.key_dim + self.value_dim

    def is_full(self, i):
        return self.layer_types[i] == "full_attention"

    @classmethod
    def from_dict(cls, cfg):
        """Accepts a flat text config or a wrapper with `text_config`
        (main.py:348-353)."""
        if "text_config" in cfg:
            tc = dict(cfg["text_config"])
            rp = tc.get("rope_parameters", {}) or {}
            tc.setdefault("rope_theta", rp.get("rope_theta", 10000000))
            tc.setdefault("partial_rotary_factor", rp.get("partial_rotary_factor", 0.25))
            cfg = tc
        names = {f.name for f in dataclasses.fields(cls)}
        return cls(**{k: v for k, v in cfg.items() if k in names})

    @classmethod
    def from_json(cls, path):
        with open(path) as f:
            return cls.from_dict(json.load(f))

    def to_dict(self):
        return dataclasses.asdict(self)


def qwen35_4b():
    """The Qwen3.5-4B text decoder shape."""
    return Qwen35Config()


def tiny(num_layers=4, hidden=256, inter=512, vocab=1024, heads=4, kv_heads=1, head_dim=256,
         lk_heads=2, lv_heads=4, lhd=128):
    """A small model of the same family for parity tests (dims keep every
    kernel's layout constraints: head dims 128/256, K % 128 == 0)."""
    return Qwen35Config(vocab_size=vocab, hidden_size=hidden, intermediate_size=inter,
                        num_hidden_layers=num_layers, num_attention_heads=heads,
                        num_key_value_heads=kv_heads, head_dim=head_dim,
                        linear_num_key_heads=lk_heads, linear_num_value_heads=lv_heads,
                        linear_key_head_dim=lhd, linear_value_head_dim=lhd)
