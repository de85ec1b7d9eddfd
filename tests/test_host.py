"""Host-side logic and the C ABI, without a GPU: config validation, the
drop-in surface, error mapping, and that libminitp.so loads and exports every
symbol include/minitp.h declares (no compute is launched)."""

import ctypes
import os
import re

import pytest
import torch

from tests.conftest import ROOT


def test_config_validation_and_heads():
    from minitp.config import ModelConfig, context_for, tiny_config

    cfg = ModelConfig(896, 4864, 24, 14, 2, 64, 151936, 1e-6, 1e6, 32768)
    cfg.validate(1)
    cfg.validate(2)
    assert cfg.local_heads(2) == (7, 1) and cfg.kv_replication(1) == 1
    with pytest.raises(ValueError, match="divisible"):
        cfg.validate(3)
    bad = ModelConfig(64, 128, 1, 8, 3, 8, 100, 1e-6, 1e4, 64)
    with pytest.raises(ValueError, match="incompatible"):
        bad.validate(2)
    assert tiny_config().vocab_size == 128
    assert context_for(1).tp_size == 1 and context_for(1).process_group is None


def test_shard_range_and_divisibility():
    from minitp.distributed.context import ParallelContext
    from minitp.parallel.linear import ColumnParallelLinear, RowParallelLinear, shard_range

    assert shard_range(10, 0, 3) == (0, 4) and shard_range(10, 1, 3) == (4, 7) and shard_range(10, 2, 3) == (7, 10)
    ctx = ParallelContext(0, 0, 2, 0, 2, torch.device("cpu"), None)
    with pytest.raises(ValueError, match="divisible"):
        ColumnParallelLinear(8, 15, ctx)
    with pytest.raises(ValueError, match="divisible"):
        RowParallelLinear(15, 8, ctx)


def test_modules_keep_reference_parameter_names_and_shapes():
    from minitp.config import ModelConfig
    from minitp.distributed.context import ParallelContext
    from minitp.layer import TPQwen2ForCausalLM

    cfg = ModelConfig(64, 128, 2, 4, 2, 16, 1000, 1e-6, 1e6, 256, True)
    m = TPQwen2ForCausalLM(cfg, ParallelContext(0, 0, 1, 0, 1, torch.device("cpu"), None))
    sd = m.state_dict()
    assert sd["model.layers.1.self_attn.qkv_proj.weight"].shape == (128, 64)
    assert sd["model.layers.1.self_attn.qkv_proj.bias"].shape == (128,)
    assert sd["model.layers.0.mlp.gate_up_proj.weight"].shape == (256, 64)
    assert sd["model.layers.0.mlp.down_proj.weight"].shape == (64, 128)
    assert sd["model.layers.0.self_attn.o_proj.weight"].shape == (64, 64)
    assert m.lm_head.weight is m.model.embed_tokens.weight
    assert {"model.norm.weight", "model.embed_tokens.weight", "lm_head.weight"} <= set(sd)


def test_cpu_forward_refuses_instead_of_falling_back():
    from minitp.config import ModelConfig
    from minitp.distributed.context import ParallelContext
    from minitp.layer import TPQwen2ForCausalLM

    cfg = ModelConfig(64, 128, 1, 4, 2, 16, 100, 1e-6, 1e4, 64, True)
    m = TPQwen2ForCausalLM(cfg, ParallelContext(0, 0, 1, 0, 1, torch.device("cpu"), None))
    with pytest.raises(RuntimeError, match="no CPU path"):
        m(torch.zeros(1, 3, dtype=torch.long))


def test_generation_state_prefill_logits_option():
    """prefill_logits is checked before anything is allocated; 'last' is the
    form generate_greedy uses, 'all' the reference's default."""
    from minitp.config import ModelConfig
    from minitp.distributed.context import ParallelContext
    from minitp.generation import GenerationState
    from minitp.layer import TPQwen2ForCausalLM

    cfg = ModelConfig(64, 128, 1, 4, 2, 16, 100, 1e-6, 1e4, 64, True)
    m = TPQwen2ForCausalLM(cfg, ParallelContext(0, 0, 1, 0, 1, torch.device("cpu"), None))
    ids = torch.zeros(1, 3, dtype=torch.long)
    for bad in ("none", "LAST", None):
        with pytest.raises(ValueError, match="prefill_logits"):
            GenerationState(m, ids, 2, prefill_logits=bad)
    assert GenerationState(m, ids, 2).prefill_logits == "all"
    st = GenerationState(m, ids, 2, prefill_logits="last")
    assert st.prefill_logits == "last"
    with pytest.raises(RuntimeError, match="no CPU path"):
        st.prefill()


def test_kv_cache_host_validation():
    from minitp.kv_cache import KVCache

    with pytest.raises(ValueError, match="init"):
        KVCache(2, 1, 2, 16, 8, torch.float32, torch.device("cpu"), init="bogus")
    kv = KVCache(2, 1, 2, 16, 8, torch.float32, torch.device("cpu"), init="zeros")
    assert kv.k[1].shape == (1, 2, 8, 16) and kv.k_buf.shape == (2, 1, 2, 8, 16)
    # capacity: max_seq_len rounded up to a power of two (multiples of 8192 past it);
    # the views keep the reference shape and every bound stays max_seq_len
    from minitp.kv_cache import cache_capacity

    assert [cache_capacity(n) for n in (1, 8, 9, 200, 384, 2560, 8192, 8193, 20000)] == \
        [1, 8, 16, 256, 512, 4096, 8192, 16384, 24576]
    kv2 = KVCache(3, 2, 2, 16, 200, torch.float32, torch.device("cpu"))
    assert kv2.capacity == 256 and kv2.k_buf.shape == (3, 2, 2, 256, 16)
    assert kv2.k[2].shape == (2, 2, 200, 16) and kv2.k[2].stride(1) == 256 * 16
    kv2.seq_len = 199
    kv2.check_room(1)
    with pytest.raises(ValueError, match="overflow"):
        kv2.check_room(2)
    assert kv.k[1].data_ptr() == kv.k_buf[1].data_ptr()  # views into one buffer
    with pytest.raises(ValueError, match="overflow"):
        kv.update(0, torch.zeros(1, 2, 9, 16), torch.zeros(1, 2, 9, 16))
    kv.poison(float("nan"))
    assert torch.isnan(kv.v[0]).all()
    kv.advance(3)
    assert kv.seq_len == 3


def test_rotary_tables_equal_reference_math_and_range_check():
    from minitp.rope import RotaryEmbedding
    from oracle.qwen2_ref import rope_tables

    rot = RotaryEmbedding(16, 1e4, 128)
    c, s = rope_tables(16, 1e4, 128)
    assert torch.equal(rot.cos_cache, c) and torch.equal(rot.sin_cache, s)
    q = torch.randn(1, 1, 1, 16)
    with pytest.raises(IndexError):
        rot.apply(q, q, torch.tensor([128 + 5]))


def test_parallel_layers_refuse_tensor_parallel_contexts():
    from minitp.distributed.context import ParallelContext
    from minitp.parallel.embedding import VocabParallelEmbedding, VocabParallelLMHead
    from minitp.parallel.linear import ColumnParallelLinear, RowParallelLinear

    ctx = ParallelContext(0, 0, 2, 0, 2, torch.device("cpu"), None)
    for make in (lambda: ColumnParallelLinear(8, 16, ctx), lambda: RowParallelLinear(16, 8, ctx),
                 lambda: VocabParallelEmbedding(16, 4, ctx), lambda: VocabParallelLMHead(4, 16, ctx)):
        with pytest.raises(NotImplementedError, match="tensor parallelism 1"):
            make()


def test_tp_greater_than_one_is_refused():
    from minitp.config import ModelConfig
    from minitp.distributed.context import ParallelContext
    from minitp.layer import TPQwen2ForCausalLM

    cfg = ModelConfig(64, 128, 1, 4, 2, 16, 100, 1e-6, 1e4, 64, True)
    with pytest.raises(NotImplementedError):
        TPQwen2ForCausalLM(cfg, ParallelContext(0, 0, 2, 0, 2, torch.device("cpu"), None))


# ---------------------------------------------------------------------------
# C ABI


def _declared_symbols():
    text = open(os.path.join(ROOT, "include", "minitp.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(minitp_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from minitp import _native

    lib = ctypes.CDLL(_native.LIB_PATH)
    names = _declared_symbols()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(names) == set(_native.SIGNATURES), set(names) ^ set(_native.SIGNATURES)


def test_abi_validation_paths_return_status_without_gpu_work():
    from minitp import _native as N

    lib = N.lib()
    assert lib.minitp_abi_version() == 5
    assert lib.minitp_status_string(N.ERR_OVERFLOW) == b"KV cache overflow"
    # K not a multiple of 8 bf16 elements: rejected before any launch
    st = lib.minitp_linear(None, N.BF16, 16, 12, 16, None, 16, 4, 1, 4, 12, N.EPI_NONE, None)
    assert st == N.ERR_ARG and b"multiple" in lib.minitp_last_error()
    with pytest.raises(ValueError, match="overflow"):
        N.check(lib.minitp_kv_write(None, N.F32, 16, 16, 16, 16, 1, 2, 4, 16, 6, 3), "kv_write")
    with pytest.raises(ValueError, match="not divisible"):
        N.check(lib.minitp_attention(None, N.F32, 16, 16, 16, 16, 1, 1, 5, 2, 16, 8, 0, 16, 1024), "attention")
    with pytest.raises(TypeError):
        N.dtype_code(torch.float16)
    assert lib.minitp_attention_workspace_bytes(1, 1, 14, 2, 64, 384) > 0
    assert lib.minitp_argmax_workspace_bytes(1, 151936) > 0


def test_add_rmsnorm_linear_parts_refuses_unserved_shapes():
    from minitp import _native as N

    lib = N.lib()
    # 17 partial rows, K past 1024, an epilogue other than SwiGLU: refused before any launch
    st = lib.minitp_add_rmsnorm_linear_parts(None, N.BF16, 16, 16, 17, 32, 16, 1e-6, 16, 16, 64, 896, N.EPI_SWIGLU)
    assert st == N.ERR_UNSUPPORTED and b"partial rows" in lib.minitp_last_error()
    st = lib.minitp_add_rmsnorm_linear_parts(None, N.BF16, 16, 16, 4, 32, 16, 1e-6, 16, 16, 64, 2048, N.EPI_SWIGLU)
    assert st == N.ERR_UNSUPPORTED
    st = lib.minitp_add_rmsnorm_linear_parts(None, N.BF16, 16, 16, 4, 32, 16, 1e-6, 16, 16, 64, 896, N.EPI_NONE)
    assert st == N.ERR_UNSUPPORTED
    with pytest.raises(ValueError, match="alias"):
        N.check(lib.minitp_add_rmsnorm_linear_parts(None, N.BF16, 16, 16, 4, 16, 16, 1e-6, 16, 16, 64, 896,
                                                    N.EPI_SWIGLU), "parts")


def test_program_create_validates_and_sizes_workspace():
    from minitp import _native as N

    lib = N.lib()
    cfg = N.Qwen2Config(N.BF16, 2, 64, 4, 2, 16, 128, 1000, 256, 1e-6)
    fake = (ctypes.c_void_p * 14)(*([4096] * 14))
    w = N.Qwen2Weights(4096, 4096, 4096, 4096, 4096, ctypes.cast(fake, ctypes.POINTER(ctypes.c_void_p)))
    h = ctypes.c_void_p()
    assert lib.minitp_qwen2_create(ctypes.byref(cfg), ctypes.byref(w), ctypes.byref(h)) == 0
    try:
        assert lib.minitp_qwen2_workspace_bytes(h, 8, 1, 24) > 0
        step = N.Qwen2Step()
        step.batch, step.tokens, step.cache_len, step.max_seq = 1, 5, 20, 24
        step.ids = step.positions = step.k_cache = step.v_cache = step.logits = step.workspace = 4096
        step.ids_ld = 5
        with pytest.raises(ValueError, match="overflow"):
            N.check(lib.minitp_qwen2_forward(h, None, ctypes.byref(step)), "forward")
        with pytest.raises(ValueError, match="tokens == 1"):
            N.check(lib.minitp_qwen2_decode(h, None, ctypes.byref(step)), "decode")
        # batch > 4 runs the GEMM LM head, which stores logits before the argmax
        step.tokens, step.cache_len, step.ids_ld, step.batch = 1, 3, 1, 8
        step.logits, step.next_tok, step.next_tok_ld = None, 4096, 1
        with pytest.raises(ValueError, match="logits buffer required"):
            N.check(lib.minitp_qwen2_decode(h, None, ctypes.byref(step)), "decode")
    finally:
        lib.minitp_qwen2_destroy(h)
    bad = N.Qwen2Config(N.BF16, 2, 64, 5, 2, 16, 128, 1000, 256, 1e-6)
    assert lib.minitp_qwen2_create(ctypes.byref(bad), ctypes.byref(w), ctypes.byref(h)) == N.ERR_ARG


def test_model_config_from_hf_dict_object_and_fallbacks():
    from types import SimpleNamespace

    from minitp.config import ModelConfig

    base = {"hidden_size": 896, "intermediate_size": 4864, "num_hidden_layers": 24, "num_attention_heads": 14,
            "num_key_value_heads": 2, "vocab_size": 151936, "rms_norm_eps": 1e-6, "max_position_embeddings": 32768}
    # transformers >= 5: theta only inside rope_parameters; no head_dim key; tie flag absent
    cfg = ModelConfig.from_hf({**base, "rope_parameters": {"rope_theta": 1000000}})
    assert cfg.head_dim == 64 and cfg.rope_theta == 1e6 and isinstance(cfg.rope_theta, float)
    assert cfg.tie_word_embeddings is True
    cfg2 = ModelConfig.from_hf(SimpleNamespace(**base, rope_theta=1e4, head_dim=128, tie_word_embeddings=False))
    assert (cfg2.head_dim, cfg2.rope_theta, cfg2.tie_word_embeddings) == (128, 1e4, False)
    with pytest.raises(KeyError):
        ModelConfig.from_hf({k: v for k, v in base.items() if k != "vocab_size"} | {"rope_theta": 1.0})
    with pytest.raises(ValueError, match="divisible"):
        ModelConfig.from_hf({**base, "rope_theta": 1.0}, tp_size=3)
    # KV heads replicate when tp exceeds them, shard otherwise
    assert cfg.kv_replication(4) == 2 and cfg.kv_replication(2) == 1 and cfg.kv_replication(1) == 1
    assert cfg.local_heads(2) == (7, 1) and cfg.local_heads(1) == (14, 2)


def test_percentiles_follow_the_reference_rank_rule():
    from minitp.bench.benchmark import percentiles

    # known answers of round(q * n) - 1 over sorted samples (benchmark.py:58-74)
    five = percentiles([5.0, 1.0, 4.0, 2.0, 3.0])
    assert (five["p50"], five["p90"], five["p99"], five["min"], five["max"]) == (2.0, 4.0, 5.0, 1.0, 5.0)
    ten = percentiles([float(i) for i in range(1, 11)])
    assert (ten["p50"], ten["p90"], ten["p99"], ten["mean"]) == (5.0, 9.0, 10.0, 5.5)
    assert percentiles([]) is None
    assert percentiles([7.0])["p99"] == 7.0


def test_bench_refuses_more_than_one_gpu():
    import json
    import subprocess
    import sys

    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in json.loads(r.stdout.strip().splitlines()[-1])["error"]
