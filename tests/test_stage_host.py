"""CPU tests of the stage trainers' host-side logic: the parts an overlapped
AdamW update is split into (`eth_amd.stage.update_parts`), checked against
parameter counts worked out by hand for a small GPT (h 64, FFN 256, 2 heads,
vocab 128, seq 32)."""

import torch

from eth_amd.model.flex_model import FlexGPTModel, middle_stage
from eth_amd.model.flex_ops import GPTConfig
from eth_amd.stage import update_parts

H, F, V, S = 64, 256, 128, 32
LN = 2 * H                      # weight + bias
QKV = H * 3 * H + 3 * H         # 12480
DENSE = H * H + H               # 4160
FC1 = H * F + F                 # 16640
FC2 = F * H + H                 # 16448
LAYER = 2 * LN + QKV + DENSE + FC1 + FC2  # 49984


def _cfg(layers):
    return GPTConfig(hidden_size=H, num_attention_heads=2, ffn_hidden_size=F, num_layers=layers, seq_length=S,
                     micro_batch_size=1, padded_vocab_size=V, params_dtype=torch.float32, device="cpu", seed=1)


def _sizes(parts):
    return [sum(p.numel() for p in part) for part in parts]


def test_middle_stage_parts_follow_the_forward():
    """Three layers: the first layer's attention half (LN1, QKV, projection,
    LN2), its MLP half (fc1, fc2) with the next layer's first LayerNorm (whose
    forward runs in the MLP half's closing bias-dropout-add), then one part
    per layer, each owning the following layer's first LayerNorm.  Every
    parameter is in exactly one part."""
    model = middle_stage(_cfg(3), 0, 3)
    parts = update_parts(model.language_model.ops)
    assert _sizes(parts) == [LN + QKV + DENSE + LN, FC1 + FC2 + LN, LAYER, LAYER - LN]
    ids = [id(p) for part in parts for p in part]
    assert len(ids) == len(set(ids)) == len(list(model.parameters()))


def test_first_last_stage_parts_put_the_embedding_first_and_the_head_last():
    """The whole model on one stage: the embedding (word and position tables)
    first, the layers as in a middle stage, and the final LayerNorm with the
    tied head copy last (read by the forward's last op)."""
    model = FlexGPTModel(_cfg(2), 0, 10 * 2 + 3)
    ops = model.language_model.ops
    assert ops[0].name == "encoder-embedding" and ops[-1].name == "gpt-post-process"
    parts = update_parts(ops)
    assert _sizes(parts) == [V * H + S * H, LN + QKV + DENSE + LN, FC1 + FC2 + LN, LAYER - LN, LN + V * H]
    assert parts[0][0] is ops[0].word_embeddings.weight
    assert any(p is ops[-1].word_embeddings.weight for p in parts[-1])
    ids = [id(p) for part in parts for p in part]
    assert len(ids) == len(set(ids)) == len(list(model.parameters()))


def test_a_stage_cut_inside_a_layer_splits_its_own_first_layer():
    """A stage starting at a layer's attention-projection op: the first
    (partial) layer still splits into its attention-side ops and its MLP
    half."""
    from eth_amd.model.flex_model import op_range_stage

    model = op_range_stage(_cfg(2), 1 + 3, 1 + 20)  # enc-attention-dense of layer 0 .. end of layer 1
    parts = update_parts(model.language_model.ops)
    assert _sizes(parts) == [DENSE + LN, FC1 + FC2 + LN, LAYER - LN]
