"""Weight loading (nanoserve/model.py:171-183 path, offline): a local HF-format folder (config.json +
sharded *.safetensors, HF tensor names) loads into Qwen2Model with every tensor bitwise equal to what was
written, the config parses through ModelConfig.from_hf_config as transformers' own Qwen2Config serialises
it, and on the GPU the loaded model's logits equal those of the model built from the same state dict."""
import json

import pytest
import torch

from nanoserve_amd.model import ModelConfig, Qwen2Model, random_state_dict

CFG = ModelConfig(vocab_size=512, hidden_size=256, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=64,
                  intermediate_size=256, rope_theta=1e6, rms_norm_eps=1e-6, tie_word_embeddings=True)


def write_folder(path, cfg, sd, shards=2):
    from safetensors.torch import save_file
    from transformers import Qwen2Config
    hf = Qwen2Config(vocab_size=cfg.vocab_size, hidden_size=cfg.hidden_size, num_hidden_layers=cfg.n_layers,
                     num_attention_heads=cfg.n_heads, num_key_value_heads=cfg.n_kv_heads,
                     intermediate_size=cfg.intermediate_size, rope_theta=cfg.rope_theta,
                     rms_norm_eps=cfg.rms_norm_eps, tie_word_embeddings=cfg.tie_word_embeddings)
    (path / "config.json").write_text(json.dumps(hf.to_dict()))
    names = sorted(sd)
    for i in range(shards):
        part = {n: sd[n].contiguous() for n in names[i::shards]}
        save_file(part, str(path / f"model-{i + 1:05d}-of-{shards:05d}.safetensors"))


def test_config_from_transformers_serialisation(tmp_path):
    write_folder(tmp_path, CFG, random_state_dict(CFG, seed=0, dtype=torch.bfloat16))
    assert ModelConfig.from_pretrained(str(tmp_path)) == CFG


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_every_tensor_loads_bitwise(tmp_path, dtype):
    sd = random_state_dict(CFG, seed=1, dtype=torch.bfloat16)
    write_folder(tmp_path, CFG, sd, shards=3)
    m = Qwen2Model.from_pretrained(str(tmp_path), device="cpu", dtype=dtype)
    assert m.cfg == CFG and m.lm_head is m.embed                      # tied LM head
    got = m.named_weights()
    assert set(got) == set(sd)
    for name, t in sd.items():
        assert got[name].dtype == dtype and torch.equal(got[name], t.to(dtype)), name
    # merged projections are views of the loaded rows (nothing stored twice)
    layer = m.layers[0]
    assert layer.q_w.data_ptr() == layer.qkv_w.data_ptr()


def test_missing_folder_raises():
    with pytest.raises(FileNotFoundError):
        Qwen2Model.from_pretrained("/nonexistent/model", device="cpu")


@pytest.mark.gpu
def test_loaded_model_runs_like_the_state_dict_model(hiplib, tmp_path):
    from nanoserve_amd.engine import LLMEngine
    sd = random_state_dict(CFG, seed=2, dtype=torch.bfloat16)
    write_folder(tmp_path, CFG, sd)
    loaded = Qwen2Model.from_pretrained(str(tmp_path), device="cuda", dtype=torch.bfloat16)
    built = Qwen2Model(CFG, {k: v.cuda() for k, v in sd.items()})
    prompt = torch.randint(0, CFG.vocab_size, (40,), generator=torch.Generator().manual_seed(3)).tolist()
    outs = []
    for m in (loaded, built):
        eng = LLMEngine(m, [], max_seq_len=128, max_num_seqs=1, batch_wait_s=0.0, kv_cache_tokens=512)
        eng.add_request(prompt, 12, ignore_eos=True)
        toks = []
        while eng.has_unfinished():
            toks += [o.token for o in eng.step()]
        outs.append(toks)
    assert outs[0] == outs[1] and len(outs[0]) == 12


def test_eos_ids_from_generation_config_with_config_fallback(tmp_path):
    """nanoserve/engine.py:33-43: generation_config.json's eos_token_id (an int or a list) first, config.json's
    when that file or key is missing or null; neither -> ValueError."""
    from nanoserve_amd.engine import load_eos_token_ids
    gen, cfg = tmp_path / "generation_config.json", tmp_path / "config.json"
    cfg.write_text(json.dumps({"model_type": "qwen2", "eos_token_id": 151643}))
    assert load_eos_token_ids(str(tmp_path)) == [151643]                     # no generation_config.json
    gen.write_text(json.dumps({"eos_token_id": [151645, 151643], "bos_token_id": 151643}))
    assert load_eos_token_ids(str(tmp_path)) == [151645, 151643]             # a list wins over config.json
    gen.write_text(json.dumps({"eos_token_id": 7}))
    assert load_eos_token_ids(str(tmp_path)) == [7]
    gen.write_text(json.dumps({"do_sample": False}))                         # key missing -> config.json
    assert load_eos_token_ids(str(tmp_path)) == [151643]
    gen.write_text(json.dumps({"eos_token_id": None}))                       # null -> config.json
    assert load_eos_token_ids(str(tmp_path)) == [151643]
    cfg.write_text(json.dumps({"model_type": "qwen2"}))
    with pytest.raises(ValueError):
        load_eos_token_ids(str(tmp_path))
    with pytest.raises(FileNotFoundError):
        load_eos_token_ids(str(tmp_path / "missing"))


@pytest.mark.gpu
def test_engines_from_a_local_folder_stop_at_its_eos(hiplib, tmp_path):
    """LLMEngine.from_pretrained / Engine.from_pretrained (nanoserve/engine.py:166-169, 311-314) on a local
    folder: weights and stop tokens both come from it. The EOS is set to the token the model emits at its
    5th step, so a request that does not ignore EOS ends there, that token included."""
    from nanoserve_amd.engine import Engine, LLMEngine
    sd = random_state_dict(CFG, seed=4, dtype=torch.bfloat16)
    write_folder(tmp_path, CFG, sd)
    prompt = torch.randint(0, CFG.vocab_size, (33,), generator=torch.Generator().manual_seed(5)).tolist()
    kw = dict(max_seq_len=128, max_num_seqs=1, batch_wait_s=0.0, kv_cache_tokens=512)
    (tmp_path / "generation_config.json").write_text(json.dumps({"eos_token_id": []}))
    free = LLMEngine(Qwen2Model(CFG, {k: v.cuda() for k, v in sd.items()}), [], **kw)
    free.add_request(prompt, 12, ignore_eos=True)
    toks = []
    while free.has_unfinished():
        toks += [o.token for o in free.step()]
    eos = toks[4]
    stop = toks.index(eos) + 1
    (tmp_path / "generation_config.json").write_text(json.dumps({"eos_token_id": [CFG.vocab_size + 1, eos]}))
    eng = LLMEngine.from_pretrained(str(tmp_path), device="cuda", dtype=torch.bfloat16, **kw)
    assert eng.eos_token_ids == [CFG.vocab_size + 1, eos]
    sid = eng.add_request(prompt, 12)
    got, finished = [], None
    while eng.has_unfinished():
        for o in eng.step():
            assert o.seq_id == sid
            got.append(o.token)
            finished = o.finished
    assert got == toks[:stop] and finished
    single = Engine.from_pretrained(str(tmp_path), device="cuda", dtype=torch.bfloat16, max_seq_len=128)
    assert list(single.generate(prompt, 12)) == toks[:stop]
    assert list(single.generate(prompt, 12, ignore_eos=True)) == toks
