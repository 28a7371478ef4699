"""Host-side argument checks of the fixed-batch runner (no GPU).

A sequence must fit its slot's run of KV blocks (``max_model_len``): a
longer one would store keys and values into the next slot's blocks and
attend to a truncated context, so prefill and decode reject it before any
device work, as the reference's block manager never hands a sequence
another sequence's blocks (nanovllm/engine/block_manager.py).
"""
import pytest
import torch
from transformers import Qwen3Config

from nv4.engine import Engine


@pytest.fixture(scope="module")
def engine():
    cfg = Qwen3Config(vocab_size=64, hidden_size=256, intermediate_size=512, num_hidden_layers=1,
                      num_attention_heads=2, num_key_value_heads=1, head_dim=128, max_position_embeddings=64,
                      rms_norm_eps=1e-6, tie_word_embeddings=False)
    return Engine(cfg, use_w4a4=False, max_num_seqs=2, max_model_len=40, block_size=16, device="cpu")


def test_prefill_rejects_overlong_and_empty_prompts(engine):
    with pytest.raises(ValueError, match="max_model_len"):
        engine.prefill(0, list(range(41)), 1.0)
    with pytest.raises(ValueError, match="max_model_len"):
        engine.prefill(0, [], 1.0)


def test_prefill_rejects_unknown_slot(engine):
    for slot in (-1, 2):
        with pytest.raises(ValueError, match="slot"):
            engine.prefill(slot, [1, 2, 3], 1.0)


def test_decode_rejects_overlong_sequences(engine):
    temps = torch.ones(2)
    with pytest.raises(ValueError, match="max_model_len"):
        engine.decode([0, 1], [1, 2], [40, 41], temps)
    with pytest.raises(ValueError, match="slot"):
        engine.decode([0, 5], [1, 2], [3, 3], temps)
    with pytest.raises(ValueError, match="one last token"):
        engine.decode([0, 1], [1], [3, 3], temps)


def test_blocks_per_slot_cover_max_model_len(engine):
    # 40 tokens in blocks of 16: three blocks per slot, slot 1 starts at block 3
    assert engine.blocks_per_seq == 3
    assert engine._slots(1, 0, 1) == [48]
