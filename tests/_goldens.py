"""Loading of the reference's golden fixtures (tests/golden/README.md) into this build's model.

The fixtures carry the reference's v2 config and v2 state-dict names. The two used here are plain
pre-norm blocks; their v3 form (modelcore/config/upgrade.py:105-126, :172-193) is written out by
hand below: block -> {mixer: attention, ffn: gated_mlp}, attn_gate -> the mixer's output_gate
feature; and state keys attn -> mixer, mlp -> ffn, attn.gate -> mixer.features.output_gate.
"""
from pathlib import Path

import torch

from modelcore_amd.model import ComponentSpec, ModelConfig

GOLDEN_DIR = Path(__file__).resolve().parent / "golden"
GOLDENS = ["v2_llama.pt", "v2_llama_kvshare_win_gated_block.pt"]


def load(name):
    return torch.load(GOLDEN_DIR / name, map_location="cpu", weights_only=True)


def v3_config(v2):
    blocks = []
    for b in v2["body"]["blocks"]:
        assert b["#type"] in ("plain_block", "gated_plain_block"), b["#type"]
        features = []
        if "attn_gate" in b:
            g = dict(b["attn_gate"])
            g.pop("#type")
            features.append(ComponentSpec("output_gate", g))
        mixer = ComponentSpec("attention", {
            "n_head": b["n_head"], "n_kv_head": b["n_kv_head"], "head_dim": b["head_dim"],
            "window": b["window"], "kv_slot": b["kv_slot"], "produces_kv": b["produces_kv"],
            "features": features})
        mlp = dict(b["mlp"])
        ffn = ComponentSpec(mlp.pop("#type"), mlp)
        blocks.append(ComponentSpec("block", {"layer_idx": b["layer_idx"], "mixer": mixer,
                                              "ffn": ffn, "features": []}))
    shared = {k: ComponentSpec(v["#type"], {p: x for p, x in v.items() if p != "#type"})
              for k, v in v2["shared"].items()}
    inp = {p: x for p, x in v2["input"].items() if p != "#type"}
    out = {p: x for p, x in v2["output"].items() if p != "#type"}
    return ModelConfig(sequence_len=v2["sequence_len"], vocab_size=v2["vocab_size"],
                       n_embd=v2["n_embd"], pad_vocab_size_to=v2["pad_vocab_size_to"],
                       shared=shared, input=ComponentSpec(v2["input"]["#type"], inp),
                       body=ComponentSpec("stack", {"blocks": blocks, "features": []}),
                       output=ComponentSpec(v2["output"]["#type"], out))


def v3_state(state):
    out = {}
    for key, value in state.items():
        parts = key.split(".")
        if len(parts) > 3 and parts[0] == "body" and parts[1] == "blocks":
            rest = ".".join(parts[3:])
            for old, new in (("attn.gate.", "mixer.features.output_gate."), ("attn.", "mixer."),
                             ("mlp.", "ffn.")):
                if rest.startswith(old):
                    rest = new + rest[len(old):]
                    break
            key = ".".join(parts[:3]) + "." + rest
        out[key] = value
    return out


def build(name, manager, device):
    """(model with the golden's weights, idx, logits)."""
    g = load(name)
    model = manager.create_model(v3_config(g["config"]), device=device, seed=0)
    missing, unexpected = model.load_state_dict(
        {k: v.to(device) for k, v in v3_state(g["state"]).items()}, strict=True)
    assert not missing and not unexpected
    return model, g["idx"], g["logits"]
