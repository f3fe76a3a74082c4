"""Checkpoint writer / reader and LoRA loader (host logic, no GPU).

The LoRA cases include the two known answers of the reference's own tests
(``tests/test_lora_loading.py:40-80``): transformer-prefixed PEFT keys with ``alpha = 4`` and
``scale = 0.5`` load onto ``transformer_blocks.0.attn.to_q`` with multiplier ``0.5 * 4 / 2``, and
Kohya flat names (``lora_unet_transformer_blocks_0_attn_to_q.lora_down.weight``) match the
same module.  The checkpoint cases pin the on-disk layout of reference
``scripts/convert_simulated.py:201-219`` / ``runtime/load.py:90-126`` (key names, dtypes,
shapes, JSON fields) and the converter's reconstruction bound.
"""
import json

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from safetensors.torch import load_file, save_file
from torch import nn

from krea2_svdquant_amd import SVDQuantLinearState
from krea2_svdquant_amd.quant import checkpoint as ck
from krea2_svdquant_amd.runtime import load as ld
from krea2_svdquant_amd.runtime import lora as lr
from krea2_svdquant_amd.runtime.linear import SVDQuantLinear
from krea2_svdquant_amd.runtime.replace import get_parent_module, iter_named_linears, replace_module
from oracle import pack as op


# ------------------------------------------------------------------------------- models
def _svdq(in_features=4, out_features=3):
    return SVDQuantLinear(SVDQuantLinearState(
        smooth_scale=torch.ones(in_features), qweight=torch.zeros(out_features, in_features // 2, dtype=torch.uint8),
        weight_scales=torch.ones(out_features, 1), l1=torch.zeros(out_features, 1), l2=torch.zeros(1, in_features),
        bias=None, group_size=in_features, original_shape=(out_features, in_features), qweight_packed=True,
        padded_in_features=in_features), backend="hip_gfx950")


class _Toy(nn.Module):
    """transformer_blocks[0].attn.to_q as an SVDQuantLinear (the reference test's toy model)."""

    def __init__(self):
        super().__init__()
        block = nn.Module()
        block.attn = nn.Module()
        block.attn.to_q = _svdq()
        self.transformer_blocks = nn.ModuleList([block])


class _Block(nn.Module):
    def __init__(self, d, ff, kv, bias):
        super().__init__()
        self.attn = nn.Module()
        self.attn.to_q = nn.Linear(d, d, bias=bias)
        self.attn.to_k = nn.Linear(d, kv, bias=bias)
        self.attn.to_v = nn.Linear(d, kv, bias=bias)
        self.attn.to_gate = nn.Linear(d, d, bias=bias)
        self.attn.to_out = nn.ModuleList([nn.Linear(d, d, bias=True), nn.Dropout(0.0)])
        self.ff = nn.Module()
        self.ff.gate = nn.Linear(d, ff, bias=bias)
        self.ff.up = nn.Linear(d, ff, bias=bias)
        self.ff.down = nn.Linear(ff, d, bias=bias)
        self.norm = nn.LayerNorm(d)


class _Transformer(nn.Module):
    """Krea2-like naming: transformer_blocks.<i>.attn.{to_q,to_k,to_v,to_gate,to_out.0}, ff.{gate,up,down}."""

    def __init__(self, blocks=3, d=128, ff=192, kv=64, seed=0):
        super().__init__()
        torch.manual_seed(seed)
        self.proj_in = nn.Linear(d, d)
        self.transformer_blocks = nn.ModuleList([_Block(d, ff, kv, bias=(i % 2 == 0)) for i in range(blocks)])


# ------------------------------------------------------------------------------- replace
def test_replace_helpers_walk_numeric_parts():
    t = _Transformer(blocks=2)
    names = [n for n, _ in iter_named_linears(t)]
    assert "transformer_blocks.0.attn.to_out.0" in names and "proj_in" not in names
    assert len(names) == 2 * 8
    parent, leaf = get_parent_module(t, "transformer_blocks.1.attn.to_out.0")
    assert leaf == "0" and parent is t.transformer_blocks[1].attn.to_out
    new = nn.Identity()
    replace_module(t, "transformer_blocks.1.attn.to_out.0", new)
    assert t.transformer_blocks[1].attn.to_out[0] is new
    replace_module(t, "transformer_blocks.0.ff.up", new)
    assert t.transformer_blocks[0].ff.up is new
    assert [n for n, _ in iter_named_linears(t, ["ff.gate"])] == ["transformer_blocks.0.ff.gate",
                                                                   "transformer_blocks.1.ff.gate"]


# ------------------------------------------------------------------------------- LoRA
def test_lora_transformer_prefixed_keys_known_answer(tmp_path):
    model = _Toy()
    down = torch.arange(8, dtype=torch.float32).reshape(2, 4) / 10
    up = torch.arange(6, dtype=torch.float32).reshape(3, 2) / 10
    f = tmp_path / "pytorch_lora_weights.safetensors"
    save_file({"transformer.transformer_blocks.0.attn.to_q.lora_A.weight": down,
               "transformer.transformer_blocks.0.attn.to_q.lora_B.weight": up,
               "transformer.transformer_blocks.0.attn.to_q.alpha": torch.tensor(4.0)}, f)
    report = lr.load_svdquant_lora_adapters(model, f, scale=0.5)
    assert report == {"lora_file": str(f), "loaded": ["transformer_blocks.0.attn.to_q"], "unmatched": [],
                      "incomplete": []}
    target = model.transformer_blocks[0].attn.to_q
    assert len(target.lora_adapters) == 1
    ad = target.lora_adapters[0]
    assert ad.multiplier == 0.5 * 4.0 / 2 and ad.rank == 2 and ad.network_alpha == 4.0
    x = torch.randn(2, 4)
    torch.testing.assert_close(ad(x), F.linear(F.linear(x, down), up) * (0.5 * 4.0 / 2))


def test_lora_flat_kohya_prefix_known_answer(tmp_path):
    model = _Toy()
    f = tmp_path / "flat.safetensors"
    save_file({"lora_unet_transformer_blocks_0_attn_to_q.lora_down.weight": torch.zeros(2, 4),
               "lora_unet_transformer_blocks_0_attn_to_q.lora_up.weight": torch.zeros(3, 2)}, f)
    report = lr.load_svdquant_lora_adapters(model, f)
    assert report["loaded"] == ["transformer_blocks.0.attn.to_q"]
    # no alpha: network_alpha defaults to the rank, multiplier = scale
    assert model.transformer_blocks[0].attn.to_q.lora_adapters[0].multiplier == 1.0


@pytest.mark.parametrize("prefix,down_sfx,up_sfx", [
    ("base_model.model.transformer_blocks.0.attn.to_q", ".lora_A.weight", ".lora_B.weight"),
    ("unet.transformer_blocks.0.attn.to_q", ".lora.down.weight", ".lora.up.weight"),
    ("transformer_blocks.0.attn.to_q", ".lora_linear_layer.down.weight", ".lora_linear_layer.up.weight"),
    ("module.diffusion_model.transformer_blocks.0.attn.to_q", ".down.weight", ".up.weight"),
    ("model.transformer.transformer_blocks.0.attn.to_q", ".lora_down.weight", ".lora_up.weight"),
])
def test_lora_key_styles(tmp_path, prefix, down_sfx, up_sfx):
    model = _Toy()
    f = tmp_path / "a.safetensors"
    save_file({prefix + down_sfx: torch.ones(3, 4), prefix + up_sfx: torch.ones(3, 3),
               prefix + ".network_alpha": torch.tensor([6.0])}, f)
    report = lr.load_svdquant_lora_adapters(model, f, scale=2.0)
    assert report["loaded"] == ["transformer_blocks.0.attn.to_q"]
    assert model.transformer_blocks[0].attn.to_q.lora_adapters[0].multiplier == 2.0 * 6.0 / 3


def test_lora_split_pairs_grammar():
    t = torch.zeros(1)
    entries = lr.group_adapters({
        "a.lora.down.weight": t, "a.lora.up.weight": t,        # ".lora.down" wins over ".down"
        "b.lora_A.weight": t,                                  # incomplete
        "c.alpha": torch.tensor([1.0, 2.0]),                   # multi-element alpha -> None
        "d.lora_alpha": torch.tensor(3.0),
        "unrelated.weight": t,
    })
    assert list(entries) == ["a", "b", "c", "d"]
    assert entries["a"].complete and entries["a"].alpha is None
    assert entries["b"].down is not None and entries["b"].up is None and not entries["b"].complete
    assert entries["c"].alpha is None and entries["c"].down is None and entries["d"].alpha == 3.0
    assert lr.parse_key("x.lora_linear_layer.down.weight") == ("x", "down")
    assert lr.parse_key("x.weight") is None
    assert lr.canonical_name("transformer.model.module.x.transformer.y") == "x.transformer.y"
    assert lr.canonical_name("transformer_blocks.0") == "transformer_blocks.0"
    root = nn.Module()
    root.blocks = nn.ModuleList([nn.Module() for _ in range(11)])
    root.blocks[0].to_q = _svdq()
    root.blocks[10].to_q = _svdq()
    index = lr.ModuleIndex(root)
    assert index.matches("lora_te_x_blocks_0_to_q") == ["blocks.0.to_q"]
    assert index.matches("blocks.10.to_q") == ["blocks.10.to_q"]
    assert index.matches("xblocks.0.to_q") == []


def test_lora_report_unmatched_incomplete_and_errors(tmp_path):
    model = _Toy()
    f = tmp_path / "mixed.safetensors"
    save_file({"transformer_blocks.0.attn.to_q.lora_A.weight": torch.zeros(2, 4),
               "transformer_blocks.0.attn.to_q.lora_B.weight": torch.zeros(3, 2),
               "transformer_blocks.0.attn.to_k.lora_A.weight": torch.zeros(2, 4),
               "transformer_blocks.0.attn.to_k.lora_B.weight": torch.zeros(3, 2),
               "transformer_blocks.0.attn.to_v.lora_A.weight": torch.zeros(2, 4)}, f)
    rep = lr.load_svdquant_lora_adapters(model, f)
    assert rep["loaded"] == ["transformer_blocks.0.attn.to_q"]
    assert rep["unmatched"] == ["transformer_blocks.0.attn.to_k"]
    assert rep["incomplete"] == ["transformer_blocks.0.attn.to_v"]
    g = tmp_path / "none.safetensors"
    save_file({"other.lora_A.weight": torch.zeros(2, 4), "other.lora_B.weight": torch.zeros(3, 2)}, g)
    with pytest.raises(ValueError, match="no LoRA tensors"):
        lr.load_svdquant_lora_adapters(_Toy(), g)
    assert lr.load_svdquant_lora_adapters(_Toy(), g, strict=False)["unmatched"] == ["other"]
    # a name that matches two modules is an error
    two = nn.Module()
    two.to_q = _svdq()
    two.attn = nn.Module()
    two.attn.to_q = _svdq()
    h = tmp_path / "two.safetensors"
    save_file({"x.attn.to_q.lora_A.weight": torch.zeros(2, 4), "x.attn.to_q.lora_B.weight": torch.zeros(3, 2)}, h)
    with pytest.raises(ValueError, match="multiple modules"):
        lr.load_svdquant_lora_adapters(two, h)
    # shape errors surface from add_lora_adapter
    bad = tmp_path / "bad.safetensors"
    save_file({"transformer_blocks.0.attn.to_q.lora_A.weight": torch.zeros(2, 5),
               "transformer_blocks.0.attn.to_q.lora_B.weight": torch.zeros(3, 2)}, bad)
    with pytest.raises(ValueError, match="down input mismatch"):
        lr.load_svdquant_lora_adapters(_Toy(), bad)


def test_lora_file_resolution(tmp_path):
    pair = {"transformer_blocks.0.attn.to_q.lora_A.weight": torch.ones(2, 4),
            "transformer_blocks.0.attn.to_q.lora_B.weight": torch.ones(3, 2)}
    d = tmp_path / "dir"
    d.mkdir()
    save_file(pair, d / "only_one.safetensors")
    assert lr.resolve_lora_file(d) == d / "only_one.safetensors"
    save_file(pair, d / "second.safetensors")
    with pytest.raises(FileNotFoundError, match="could not infer"):
        lr.resolve_lora_file(d)
    save_file(pair, d / "adapter_model.safetensors")
    assert lr.resolve_lora_file(d) == d / "adapter_model.safetensors"
    assert lr.resolve_lora_file(d, weight_name="second.safetensors") == d / "second.safetensors"
    with pytest.raises(FileNotFoundError):
        lr.resolve_lora_file(d, weight_name="absent.safetensors")
    with pytest.raises(FileNotFoundError):
        lr.resolve_lora_file(tmp_path / "no_such_file.safetensors")
    # .bin files are read with weights_only=True, including a {"state_dict": ...} wrapper
    b = tmp_path / "bin"
    b.mkdir()
    torch.save({"state_dict": dict(pair, step=torch.tensor(3))}, b / "pytorch_lora_weights.bin")
    model = _Toy()
    rep = lr.load_svdquant_lora_adapters(model, b)
    assert rep["loaded"] == ["transformer_blocks.0.attn.to_q"] and rep["lora_file"].endswith(".bin")


# ------------------------------------------------------------------------------- checkpoint
def _convert(tmp_path, **kw):
    t = _Transformer(**{k: kw.pop(k) for k in ("blocks", "d", "ff", "kv") if k in kw})
    absmax = kw.pop("absmax", None)
    meta = ck.convert_transformer(t, tmp_path / "ckpt", absmax=absmax, log=None, seed=5, **kw)
    return t, meta


def test_checkpoint_layout_matches_reference_format(tmp_path):
    t, meta = _convert(tmp_path, group_size=64, rank=16, attn_rank=8, mlp_rank=16,
                       absmax={"transformer_blocks.1.attn.to_q": torch.rand(128) * 10})
    root = tmp_path / "ckpt"
    assert (root / "README.md").exists()
    disk = json.loads((root / "svdquant_config.json").read_text())
    assert disk == meta
    assert disk["format"] == "krea2-svdquant-transformer-v1" and disk["group_size"] == 64
    assert disk["num_blocks"] == 3 and disk["calibrated"] is True and len(disk["layers"]) == 24
    assert set(disk["options"]) == {"rank", "attn_rank", "mlp_rank", "skip_first_blocks", "skip_last_blocks",
                                    "skip_qk", "max_layers", "svd_oversample", "svd_niter", "svd_exact"}
    assert disk["layers"]["transformer_blocks.1.attn.to_q"] == {"rank": 8, "group_size": 64, "shape": [128, 128],
                                                                "calibrated": True}
    assert disk["layers"]["transformer_blocks.0.ff.down"]["rank"] == 16
    assert disk["layers"]["transformer_blocks.0.ff.down"]["shape"] == [128, 192]
    tensors = load_file(str(root / "transformer_svdquant.safetensors"))
    for name, lm in disk["layers"].items():
        key = name.replace(".", "__")
        n, k = lm["shape"]
        r = lm["rank"]
        kp = -(-k // 64) * 64
        assert tensors[f"{key}.qweight_packed"].dtype == torch.uint8
        assert tuple(tensors[f"{key}.qweight_packed"].shape) == (n, kp // 2)
        assert tensors[f"{key}.weight_scales"].dtype == torch.float16
        assert tuple(tensors[f"{key}.weight_scales"].shape) == (n, kp // 64)
        assert tensors[f"{key}.smooth_scale"].dtype == torch.bfloat16 and tuple(tensors[f"{key}.smooth_scale"].shape) == (k,)
        assert tensors[f"{key}.l1"].dtype == torch.bfloat16 and tuple(tensors[f"{key}.l1"].shape) == (n, r)
        assert tensors[f"{key}.l2"].dtype == torch.bfloat16 and tuple(tensors[f"{key}.l2"].shape) == (r, k)
        dense = get_parent_module(t, name)
        mod = getattr(dense[0], dense[1]) if not dense[1].isdigit() else dense[0][int(dense[1])]
        assert (f"{key}.bias" in tensors) == (mod.bias is not None)
    # uncalibrated layers use identity smoothing
    assert torch.all(tensors["transformer_blocks__0__attn__to_q.smooth_scale"] == 1)
    assert not torch.all(tensors["transformer_blocks__1__attn__to_q.smooth_scale"] == 1)


def test_converter_reconstruction_bound(tmp_path):
    """W*s = dequant(codes) + L1 L2 up to half a quantization step per element (codes come from
    fp32 scales that are stored in fp16, hence the small slack), checked with the oracle's unpacker."""
    t, meta = _convert(tmp_path, blocks=1, group_size=64, rank=16, attn_rank=16, mlp_rank=16,
                       absmax={"transformer_blocks.0.ff.up": torch.rand(128) * 5 + 0.1})
    tensors = load_file(str(tmp_path / "ckpt" / "transformer_svdquant.safetensors"))
    for name in ("transformer_blocks.0.ff.up", "transformer_blocks.0.ff.down", "transformer_blocks.0.attn.to_k"):
        key = name.replace(".", "__")
        parent, leaf = get_parent_module(t, name)
        w = getattr(parent, leaf).weight.detach().to(torch.bfloat16).float()
        s = tensors[f"{key}.smooth_scale"].float()
        target = (w * s).to(torch.bfloat16).float()
        n, k = w.shape
        q = op.unpack_int4(tensors[f"{key}.qweight_packed"].numpy(), k).astype(np.float32)
        sc = tensors[f"{key}.weight_scales"].float().numpy()
        deq = q * np.repeat(sc, 64, axis=1)[:, :k]
        low = (tensors[f"{key}.l1"].float() @ tensors[f"{key}.l2"].float()).numpy()
        err = np.abs(deq + low - target.numpy())
        bound = np.repeat(sc, 64, axis=1)[:, :k] * (0.5 + 8 * 2.0 ** -10) + 1e-7
        assert np.all(err <= bound), name
        assert np.abs(q).max() <= 8


def test_checkpoint_round_trip_into_fresh_model(tmp_path):
    _, meta = _convert(tmp_path, group_size=64, rank=16, attn_rank=8, mlp_rank=16, skip_first_blocks=1,
                       skip_qk=True)
    assert "transformer_blocks.0.attn.to_v" not in meta["layers"]
    assert "transformer_blocks.2.attn.to_q" not in meta["layers"] and "transformer_blocks.2.attn.to_k" not in meta["layers"]
    fresh = _Transformer()
    cfg = ld.load_svdquant_transformer(fresh, tmp_path / "ckpt", backend="hip_gfx950")
    rep = cfg["_load_report"]
    assert rep["replaced"] == list(meta["layers"]) and rep["missing"] == []
    tensors = load_file(str(tmp_path / "ckpt" / "transformer_svdquant.safetensors"))
    for name in meta["layers"]:
        parent, leaf = get_parent_module(fresh, name)
        mod = parent[int(leaf)] if leaf.isdigit() else getattr(parent, leaf)
        assert isinstance(mod, SVDQuantLinear) and mod.backend.value == "hip_gfx950"
        st = mod.state
        key = name.replace(".", "__")
        assert torch.equal(st.qweight, tensors[f"{key}.qweight_packed"]) and st.qweight_packed
        assert torch.equal(st.weight_scales, tensors[f"{key}.weight_scales"])
        assert torch.equal(st.l1, tensors[f"{key}.l1"]) and torch.equal(st.l2, tensors[f"{key}.l2"])
        assert st.group_size == 64 and st.original_shape == tuple(meta["layers"][name]["shape"])
        assert st.padded_in_features == 2 * tensors[f"{key}.qweight_packed"].shape[1]
    assert isinstance(fresh.transformer_blocks[0].attn.to_q, nn.Linear)
    assert isinstance(fresh.transformer_blocks[1].attn.to_out[0], SVDQuantLinear)
    assert isinstance(fresh.proj_in, nn.Linear)
    # max_layers / skip_last_blocks
    ck.convert_transformer(_Transformer(), tmp_path / "c2", max_layers=3, log=None)
    assert len(json.loads((tmp_path / "c2" / "svdquant_config.json").read_text())["layers"]) == 3
    m3 = ck.convert_transformer(_Transformer(), tmp_path / "c3", skip_last_blocks=2, log=None, group_size=64)
    assert {ck.block_index(n) for n in m3["layers"]} == {0}


def _write_checkpoint(root, layers, tensors, group_size=None):
    root.mkdir(parents=True, exist_ok=True)
    cfg = {"layers": layers}
    if group_size is not None:
        cfg["group_size"] = group_size
    (root / "svdquant_config.json").write_text(json.dumps(cfg))
    save_file(tensors, str(root / "transformer_svdquant.safetensors"))


def _layer_tensors(key, n=6, k=100, r=2, g=32, bias=False):
    kp = -(-k // g) * g
    rng = np.random.default_rng(1)
    q = rng.integers(-8, 8, size=(n, kp)).astype(np.int8)
    t = {f"{key}.qweight_packed": torch.from_numpy(op.pack_int4(q)),
         f"{key}.weight_scales": torch.rand(n, kp // g).to(torch.float16),
         f"{key}.smooth_scale": torch.rand(k).to(torch.bfloat16),
         f"{key}.l1": torch.randn(n, r).to(torch.bfloat16), f"{key}.l2": torch.randn(r, k).to(torch.bfloat16)}
    if bias:
        t[f"{key}.bias"] = torch.randn(n).to(torch.bfloat16)
    return t


def test_loader_rules_missing_group_and_shapes(tmp_path):
    def model():
        m = nn.Module()
        m.blocks = nn.ModuleList([nn.Module()])
        m.blocks[0].proj = nn.Linear(100, 6)
        m.blocks[0].out = nn.Linear(100, 6)
        return m

    # group size: layer entry, else file entry, else 128
    for layer_g, file_g, want in ((32, 64, 32), (None, 32, 32), (None, None, 128)):
        root = tmp_path / f"g{layer_g}{file_g}"
        meta = {"shape": [6, 100]} if layer_g is None else {"shape": [6, 100], "group_size": layer_g}
        _write_checkpoint(root, {"blocks.0.proj": meta}, _layer_tensors("blocks__0__proj", g=want, bias=True), file_g)
        m = model()
        ld.load_svdquant_transformer(m, root, backend="hip_gfx950")
        st = m.blocks[0].proj.state
        assert st.group_size == want and st.padded_in_features == -(-100 // want) * want
        assert st.bias is not None and st.original_shape == (6, 100)
    # a missing tensor: KeyError when strict, skipped and reported otherwise
    t = _layer_tensors("blocks__0__proj")
    t.update(_layer_tensors("blocks__0__out"))
    del t["blocks__0__out.l2"]
    root = tmp_path / "missing"
    _write_checkpoint(root, {"blocks.0.proj": {"shape": [6, 100]}, "blocks.0.out": {"shape": [6, 100]}}, t, 32)
    with pytest.raises(KeyError, match="blocks.0.out"):
        ld.load_svdquant_transformer(model(), root)
    m = model()
    rep = ld.load_svdquant_transformer(m, root, strict=False)["_load_report"]
    assert rep["replaced"] == ["blocks.0.proj"] and rep["missing"] == ["blocks__0__out.l2"]
    assert isinstance(m.blocks[0].out, nn.Linear) and isinstance(m.blocks[0].proj, SVDQuantLinear)
    # inconsistent shapes fail at load, naming the layer
    root = tmp_path / "bad"
    _write_checkpoint(root, {"blocks.0.proj": {"shape": [6, 128]}}, _layer_tensors("blocks__0__proj"), 32)
    with pytest.raises(ValueError, match="blocks.0.proj"):
        ld.load_svdquant_transformer(model(), root)
    with pytest.raises(FileNotFoundError):
        ld.load_svdquant_transformer(model(), tmp_path / "nowhere")
    assert ld._resolve_checkpoint_dir(tmp_path / "nowhere") == tmp_path / "nowhere"
    assert ld._layer_key("transformer_blocks.3.attn.to_out.0") == "transformer_blocks__3__attn__to_out__0"
