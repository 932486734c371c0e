"""Host-only checks of the decode driver's launch planning (kcModelPlanDecode): no GPU needed.

The fused single-token path (six kernels per layer) must have a launch shape at the widths of the
common Llama / Qwen3 families, including FFN widths whose super-block group count is a prime above
the wavefront cap (Llama-2-7B's 11008: 11 groups; Qwen3-14B's 17408: 17 groups), and the config
check must refuse what the kernels cannot run (head_dim below 32: the batch attention kernel
splits a head row over 16 lanes in pairs)."""
import pytest

import kernelcore_amd as kc


def cfg(**over):
    c = dict(n_layer=2, n_embd=4096, n_head=32, n_head_kv=8, head_dim=128, n_ff=11008, n_vocab=32000,
             norm_eps=1e-5, rope_theta=1e4, rope_neox=0, qk_norm=0, max_ctx=512, max_batch=64)
    c.update(over)
    return c


@pytest.mark.parametrize("n_embd,n_head,n_head_kv,n_ff", [
    (4096, 32, 32, 11008),   # Llama-2-7B
    (5120, 40, 8, 17408),    # Qwen3-14B
    (5120, 64, 8, 25600),    # Qwen3-32B
    (3072, 24, 8, 8192),     # Llama-3.2-3B (config 4)
    (4096, 32, 8, 12288),    # Qwen3-8B (config 5)
    (4096, 32, 8, 14336),    # Llama-3.1-8B
    (2048, 32, 8, 8192),     # Llama-3.2-1B (head_dim 64 below)
])
def test_fused_decode_has_a_launch_shape(n_embd, n_head, n_head_kv, n_ff):
    hd = n_embd // n_head if n_embd // n_head in (64, 128) else 128
    assert kc.plan_decode(**cfg(n_embd=n_embd, n_head=n_head, n_head_kv=n_head_kv, head_dim=hd, n_ff=n_ff)) == 1


def test_unfused_fallback_for_wide_inputs():
    # n_embd 32768: the norm prologue's staging registers cannot hold the row; the driver still
    # accepts the config and decodes with one kernel per op
    assert kc.plan_decode(**cfg(n_embd=32768, n_head=256, n_ff=8192)) == 0


@pytest.mark.parametrize("hd", [16, 48, 96])
def test_head_dim_limits(hd):
    with pytest.raises(kc.KcError) as e:
        kc.plan_decode(**cfg(n_head=4096 // hd if 4096 % hd == 0 else 32, head_dim=hd))
    assert e.value.name == "InvalidValue"


def test_head_dim_32_and_256_accepted():
    assert kc.plan_decode(**cfg(n_head=128, n_head_kv=32, head_dim=32)) in (0, 1)
    assert kc.plan_decode(**cfg(n_head=16, n_head_kv=8, head_dim=256)) in (0, 1)
