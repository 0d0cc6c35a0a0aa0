"""The decode bandwidth ceiling (x0ne-core/runtime/src/roofline.rs:1-102): at batch b each step
reads every weight once and each sequence's K and V once, so tok/s <= b * bandwidth / bytes."""
from __future__ import annotations

from dataclasses import dataclass

MI355X_HBM_GBS = 8000.0  # published peak, decimal GB/s


@dataclass(frozen=True)
class Shape:
    hidden: int
    inter: int
    layers: int
    q_heads: int
    kv_heads: int
    head_dim: int
    vocab: int
    tied: bool = False

    @staticmethod
    def of(config: dict) -> "Shape":
        return Shape(config["hidden_size"], config["intermediate_size"], config["num_hidden_layers"],
                     config["num_attention_heads"], config["num_key_value_heads"], config["head_dim"],
                     config["vocab_size"], bool(config.get("tie_word_embeddings", False)))

    @property
    def q_dim(self):
        return self.q_heads * self.head_dim

    @property
    def kv_dim(self):
        return self.kv_heads * self.head_dim


def linear_params_per_layer(s: Shape) -> int:
    """config.rs:150-159: h (q + 2 kv) + q h + 3 h inter."""
    return s.hidden * (s.q_dim + 2 * s.kv_dim) + s.q_dim * s.hidden + 3 * s.hidden * s.inter


def norm_params_per_layer(s: Shape) -> int:
    """config.rs:161-165: two h-norms and the two head-dim QK norms."""
    return 2 * s.hidden + 2 * s.head_dim


def weight_bytes_per_token(s: Shape) -> int:
    """roofline.rs:55-61: every layer weight and norm, one embedding row, the final norm and the LM
    head (the embedding itself when tied), bf16."""
    per_layer = linear_params_per_layer(s) + norm_params_per_layer(s)
    return 2 * (s.layers * per_layer + s.hidden + s.vocab * s.hidden + s.hidden)


def kv_bytes_per_position(s: Shape) -> int:
    """config.rs:167-170: K and V of every layer, bf16."""
    return s.layers * 4 * s.kv_dim


def mean_decode_ctx(prompt: int, generated: int) -> float:
    """roofline.rs:92-96: decode measured as (n - 1) / (t_n - t_1) attends prompt + n / 2 on average."""
    return prompt + generated / 2.0


def step_bytes(s: Shape, ctx: float, batch: int = 1) -> float:
    return weight_bytes_per_token(s) + batch * kv_bytes_per_position(s) * ctx


def ceiling_tok_s(s: Shape, ctx: float, batch: int = 1, bandwidth_gbs: float = MI355X_HBM_GBS) -> float:
    return batch * bandwidth_gbs * 1e9 / step_bytes(s, ctx, batch)


def gemv_bytes(rows: int, cols: int, out_bytes: int = 2, in_bytes: int = 2) -> int:
    """Algorithmic bytes of one y = W x: the bf16 weights, the input row, the output row."""
    return rows * cols * 2 + cols * in_bytes + rows * out_bytes
