"""``run.py``: the reference's command line (examples/qwen3_1_7b-tilelang/run.py:
61-97) over the HIP engines.

On the CPU: the argument rules, the engine a checkpoint's ``model_type`` picks,
and the refusal to run anywhere but on a GPU (there is no CPU path).  On the GPU:
a text prompt through a self-written checkpoint and its tokenizer -- the tokens
must be those the engine gives from the same weights drawn in memory, bit for
bit -- and the synthetic-weight mode.
"""
import json

import pytest
import torch

import run as R
from tilefoundry_amd.qwen3 import TINY, synthetic_weights
from tilefoundry_amd.qwen3.engine import Engine

CFG = TINY.with_(dtype=torch.bfloat16)


def test_arguments_need_a_weight_source_and_a_prompt():
    for argv in (["--random-prompt", "4"], ["--synthetic", "c1"],
                 ["--synthetic", "c1", "--ckpt", "x", "--random-prompt", "4"],
                 ["--synthetic", "c1", "--prompt-ids", "1", "--random-prompt", "4"]):
        with pytest.raises(SystemExit):
            R.main(argv)


def test_model_type_picks_the_engine(tmp_path):
    class A:
        model = None
        ckpt = tmp_path
    for kind, want in (("qwen3", "qwen3"), ("qwen3_5_moe", "qwen3_5"),
                       ("qwen3_5_moe_text", "qwen3_5"), ("granitemoehybrid", "granite")):
        (tmp_path / "config.json").write_text(json.dumps({"model_type": kind}))
        assert R.model_of(A) == want
    (tmp_path / "config.json").write_text(json.dumps({"model_type": "llama"}))
    with pytest.raises(SystemExit):
        R.model_of(A)


def test_no_cpu_path(monkeypatch):
    monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
    with pytest.raises(SystemExit, match="no GPU"):
        R.main(["--synthetic", "c1", "--random-prompt", "4", "--max-new-tokens", "2"])


def _checkpoint(tmp_path, w):
    from tokenizers import Tokenizer, models, pre_tokenizers
    from transformers import PreTrainedTokenizerFast

    from tests.test_checkpoint import _qwen3_hf

    _qwen3_hf(CFG, w).save_pretrained(tmp_path)
    tok = Tokenizer(models.WordLevel({f"w{i}": i for i in range(CFG.vocab_size)}, unk_token="w0"))
    tok.pre_tokenizer = pre_tokenizers.Whitespace()
    PreTrainedTokenizerFast(tokenizer_object=tok, unk_token="w0").save_pretrained(tmp_path)


@pytest.mark.gpu
def test_text_prompt_through_a_checkpoint(gpu_device, tmp_path, capsys):
    w = synthetic_weights(CFG, seed=11, norms="ones")
    _checkpoint(tmp_path, w)
    prompt = [5, 17, 300, 4095, 2, 9]
    print(f"[run] checkpoint at {tmp_path}", flush=True)
    capsys.readouterr()
    assert R.main(["--ckpt", str(tmp_path), "--prompt", " ".join(f"w{t}" for t in prompt),
                   "--max-new-tokens", "24", "--device", gpu_device, "--mode", "persistent"]) == 0
    out = capsys.readouterr().out.splitlines()
    got = [int(t[1:]) for t in out[0].split()]
    want = Engine(CFG, w, device=gpu_device, max_new=24, prompt_room=64,
                  mode="persistent").generate(prompt, 24).tokens
    assert got == want
    assert "tok/s (24 tokens in" in out[2] and "prompt 6 tokens" in out[3]


@pytest.mark.gpu
def test_synthetic_weights_and_random_prompt(gpu_device, capsys):
    assert R.main(["--synthetic", "c1", "--random-prompt", "8", "--max-new-tokens", "16",
                   "--device", gpu_device]) == 0
    out = capsys.readouterr().out.splitlines()
    assert len(out[0].split()) == 16 and all(0 <= int(t) < CFG.vocab_size for t in out[0].split())
    assert "qwen3 (persistent)" in out[3]          # C1's shape is not the XCD kernel's


def test_sampling_flags():
    """--temperature / --top-k / --top-p need --sample; --sample takes each model's
    reference defaults, which the flags override; out-of-range values refuse."""
    with pytest.raises(SystemExit, match="need --sample"):
        R.main(["--synthetic", "c1", "--random-prompt", "4", "--top-k", "5"])

    class A:
        sample, temperature, top_k, top_p, sample_seed = True, None, None, None, 3
    s = R.sampling_of(A, "qwen3_5")
    assert (s.temperature, s.top_k, s.top_p, s.seed) == (1.0, 20, 0.95, 3)
    s = R.sampling_of(A, "granite")
    assert (s.top_k, s.top_p) == (0, 1.0)
    A.temperature, A.top_k = 0.5, 8
    s = R.sampling_of(A, "granite")
    assert (s.temperature, s.top_k) == (0.5, 8)
    A.top_k = 65
    with pytest.raises(ValueError):
        R.sampling_of(A, "qwen3")
    A.sample = False
    assert R.sampling_of(A, "qwen3") is None


@pytest.mark.gpu
def test_sampled_run_is_the_batch_engine_with_one_sequence(gpu_device, capsys):
    """--sample on Qwen3 runs the batched engine with one sequence: its tokens are
    those BatchEngine gives with the same sampling, and a second seed differs."""
    from tilefoundry_amd.qwen3.batch_engine import BatchEngine
    from tilefoundry_amd.sampling import Sampling

    argv = ["--synthetic", "c1", "--prompt-ids", "5,17,300,9", "--max-new-tokens", "16",
            "--device", gpu_device, "--sample", "--top-k", "20", "--temperature", "1.3"]
    assert R.main(argv + ["--sample-seed", "7"]) == 0
    out = capsys.readouterr().out.splitlines()
    got = [int(t) for t in out[0].split()]
    assert "qwen3 (batch, sampled)" in out[3]
    w = synthetic_weights(CFG, seed=0)
    eng = BatchEngine(CFG, w, batch=1, device=gpu_device, max_new=16, prompt_room=64,
                      sampling=Sampling(temperature=1.3, top_k=20, top_p=0.95, seed=7))
    assert got == eng.generate([[5, 17, 300, 9]], 16).tokens[0]
    assert R.main(argv + ["--sample-seed", "8"]) == 0
    assert [int(t) for t in capsys.readouterr().out.splitlines()[0].split()] != got
