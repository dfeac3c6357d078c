"""The host mirror's dtype and precision rules, on the CPU: every refusal here comes before any
device call, so tensors are stand-ins that carry only a shape and a dtype.

The reference's own rules (noetic-tensor 0.7.0):
- `log_softmax` (activation.rs:30-42) on bf16/f16 logits fails `same_dtype` at `x.sub(max)`
  because `max_dim` computes 16-bit values in f32 into f32 storage (float.rs:43-58, 710-722):
  "sub: bf16 and f32 (casts are explicit)" (infer.rs:157-158). So `token_log_probs`,
  `categorical_kl` and `categorical_entropy` refuse untempered 16-bit logits.
- `tempered_logits` (rl.rs:475-486) divides unless τ == 1 (`div_scalar` makes 16-bit logits f32,
  float.rs:494-499), then adds the f32 mask: at τ == 1 a 16-bit tensor with a mask fails
  "add: bf16 and f32".
- `sample_categorical` (rl.rs:510-529) adds f32 Gumbel noise to the tempered logits at τ > 0
  (`from_f64s` computes 16-bit dtypes in f32, float.rs:257-260): bf16 at τ == 1 fails
  "add: bf16 and f32" after the row check; τ == 0 with a mask fails in tempered_logits.
- `Tensor::matmul` on a GPU runs at the thread's `matmul_precision()` (float.rs:924-930,
  precision.rs:49-63); the readout fusion is the Half product, so the mirror refuses it at F32.
The fused entries (`sample_logp`, `score` with a `Tempered` triple, the readout entries) take
16-bit logits at every τ, widened exactly: the reference's chain on `logits.cast(F32)`."""
import threading

import pytest

import noetic_ops as nops
import noetic_rl as nr


class Stub:
    """A tensor's shape and dtype, with no storage."""

    def __init__(self, shape, dtype):
        self.shape = tuple(shape)
        self.dtype = dtype
        self.numel = 1
        for s in self.shape:
            self.numel *= s

    @property
    def ptr(self):
        raise AssertionError("a refusal under test reached a device call")


SUB = "sub: bf16 and f32 (casts are explicit)"
ADD = "add: bf16 and f32 (casts are explicit)"


def test_tempered_dtype_follows_the_reference():
    td = nr.tempered_dtype
    assert td("f32", 1.0, None) == "f32" and td("f32", 0.7, "f32") == "f32" and td("f32", 1.0, "u8") == "f32"
    assert td("bf16", 1.0, None) == "bf16" and td("f16", 1.0, None) == "f16"
    assert td("bf16", 0.7, None) == "f32" and td("bf16", 0.7, "u8") == "f32" and td("f16", 2.0, "f32") == "f32"
    # a 16-bit additive mask of the logits' dtype on untempered 16-bit logits adds, computing in
    # f32 into f32 storage (fdisp, float.rs:43-58; f32_operand on a GPU)
    assert td("bf16", 1.0, "bf16") == "f32" and td("f16", 1.0, "f16") == "f32"
    with pytest.raises(nr.DTypeError, match="add: bf16 and f16"):
        td("bf16", 1.0, "f16")
    with pytest.raises(nr.DTypeError, match=ADD.replace("(", r"\(").replace(")", r"\)")):
        td("bf16", 1.0, "u8")
    with pytest.raises(nr.DTypeError, match="add: f16 and f32"):
        td("f16", 1.0, "f32")
    with pytest.raises(nr.DTypeError, match="add: f32 and bf16"):
        td("bf16", 0.5, "bf16")  # the divided logits are f32, the mask is not
    assert issubclass(nr.DTypeError, TypeError)


def test_reference_named_functions_refuse_16_bit_logits_where_the_reference_does():
    x4 = Stub((2, 3, 4, 50), "bf16")
    tok = Stub((2, 3, 4), "i32")
    keep = Stub((2, 3, 4, 50), "u8")
    with pytest.raises(nr.DTypeError) as e:
        nr.token_log_probs(x4, tok)
    assert str(e.value) == SUB
    with pytest.raises(nr.DTypeError) as e:
        nr.token_log_probs(nr.tempered_logits(x4, 1.0), tok)  # τ == 1 without a mask: no divide
    assert str(e.value) == SUB
    with pytest.raises(nr.DTypeError) as e:
        nr.tempered_logits(x4, 1.0, keep)
    assert str(e.value) == ADD
    assert nr.tempered_logits(x4, 0.7, keep).dtype == "f32"
    with pytest.raises(nr.DTypeError) as e:
        nr.categorical_entropy(x4)
    assert str(e.value) == SUB
    with pytest.raises(nr.DTypeError) as e:
        nr.categorical_kl(Stub((2, 3, 4, 50), "f32"), x4)  # the reference side's log_softmax
    assert str(e.value) == SUB
    with pytest.raises(nr.DTypeError) as e:
        nr.reference_kl(x4, x4, 1.0, None)
    assert str(e.value) == SUB
    with pytest.raises(nr.DTypeError) as e:
        nr.reference_kl(x4, x4, 1.0, keep)
    assert str(e.value) == ADD
    with pytest.raises(nr.DTypeError) as e:
        nr.sample_categorical(x4, 0.0, keep, None)  # greedy tempers at τ = 1
    assert str(e.value) == ADD
    with pytest.raises(nr.DTypeError) as e:
        nr.sample_categorical(Stub((2, 3, 4, 50), "f16"), 1.0, keep, None)
    assert str(e.value) == "add: f16 and f32 (casts are explicit)"
    # the materialised op sequence refuses in the same place
    with pytest.raises(nr.DTypeError) as e:
        nops.tempered_logits(x4, 1.0, Stub((1, 1, 1, 50), "f32"))
    assert str(e.value) == ADD
    # a bf16 additive mask on untempered bf16 logits: tempered_logits' result is f32, so the
    # reference's functions take it, and sampling at τ == 1 adds f32 noise to f32 (no refusal
    # before the device)
    m16 = Stub((2, 3, 4, 50), "bf16")
    assert nr.tempered_logits(x4, 1.0, m16).dtype == "f32"
    for call in (lambda: nr.sample_categorical(x4, 1.0, m16, None),
                 lambda: nr.sample_categorical(x4, 0.0, m16, None),
                 lambda: nr.token_log_probs(nr.tempered_logits(x4, 1.0, m16), tok)):
        with pytest.raises((AssertionError, nr.HipUnavailable)):  # past the dtype checks, at the device
            call()
    with pytest.raises(nr.DTypeError) as e:
        nr.tempered_logits(x4, 0.7, m16)  # the divided logits are f32, the mask is not
    assert str(e.value) == "add: f32 and bf16 (casts are explicit)"
    # shape checks come first, as in the reference
    with pytest.raises(ValueError, match="tokens shape"):
        nr.token_log_probs(x4, Stub((2, 3), "i32"))
    with pytest.raises(ValueError, match="mask rank"):
        nops.tempered_logits(x4, 1.0, Stub((1, 50), "f32"))


def test_the_readout_fusion_is_gated_on_half_precision():
    h = Stub((4, 64), "f32")
    assert nr.matmul_precision() == nr.MatmulPrecision.F32  # the reference's default
    with pytest.raises(ValueError, match="MatmulPrecision::Half"):
        nr.readout_sample_logp(h, None, 0.7, None, None)
    with pytest.raises(ValueError, match="MatmulPrecision::Half"):
        nr.readout_score(h, None, 0.7, None, None)
    with nr.matmul_precision_scope(nr.MatmulPrecision.HALF):
        assert nr.matmul_precision() == nr.MatmulPrecision.HALF
        seen = []
        t = threading.Thread(target=lambda: seen.append(nr.matmul_precision()))
        t.start()
        t.join()
        assert seen == [nr.MatmulPrecision.F32]  # per thread, as precision.rs keeps it
    assert nr.matmul_precision() == nr.MatmulPrecision.F32
    assert nr.set_matmul_precision(nr.MatmulPrecision.HALF) == nr.MatmulPrecision.F32
    assert nr.set_matmul_precision(nr.MatmulPrecision.F32) == nr.MatmulPrecision.HALF
    assert nops.MatmulPrecision is nr.MatmulPrecision


class PackedStub:
    """A packed head's shape and original dtype, with no storage."""

    def __init__(self, dim, vocab, dtype):
        self.dim, self.vocab, self.weight_dtype, self.batched, self.seeds = dim, vocab, dtype, False, 1

    def seed_ptr(self, seed):
        raise AssertionError("a refusal under test reached a device call")


def test_the_readout_fusion_takes_one_dtype_as_matmul_does():
    # x.matmul(w) checks the shapes, then same_dtype (float.rs:946-949): mixed hidden and head
    # dtypes are refused before any device call, whatever the pair
    with nr.matmul_precision_scope(nr.MatmulPrecision.HALF):
        for hd, wd in (("f32", "bf16"), ("bf16", "f32"), ("f16", "bf16"), ("f32", "f16")):
            with pytest.raises(nr.DTypeError) as e:
                nr.readout_sample_logp(Stub((4, 64), hd), PackedStub(64, 300, wd), 0.7, None, None)
            assert str(e.value) == f"matmul: {hd} and {wd} (casts are explicit)"
            with pytest.raises(nr.DTypeError):
                nr.readout_score(Stub((4, 64), hd), PackedStub(64, 300, wd), 0.7, None, None)
        # the shape check comes first
        with pytest.raises(ValueError, match="d 32 against the weight's 64"):
            nr.readout_sample_logp(Stub((4, 32), "f32"), PackedStub(64, 300, "bf16"), 0.7, None, None)


def test_per_token_functions_keep_the_reference_dtype_rules():
    """The losses and estimators meet their operands in the reference's binary ops (same_dtype):
    policy_gradient_loss's logp · w (rl.rs:232), the log-ratio logp − old (rl.rs:240) and PPO's
    r · A with r computed in f32 (rl.rs:270), kl_estimate's ref_logp − logp (rl.rs:392). Other
    pairings, a 16-bit mask, and 16-bit operands of one dtype pass to the device (widened there)."""
    f32, b16, h16 = (lambda d: Stub((2, 3, 4), d))("f32"), Stub((2, 3, 4), "bf16"), Stub((2, 3, 4), "f16")
    clip = nr.Clip.symmetric(0.2)
    msg = lambda e: str(e.value)
    with pytest.raises(nr.DTypeError) as e:
        nr.policy_gradient_loss(f32, b16)
    assert msg(e) == "mul: f32 and bf16 (casts are explicit)"
    with pytest.raises(nr.DTypeError) as e:
        nr.clipped_policy_loss(b16, f32, f32, None, clip)
    assert msg(e) == "sub: bf16 and f32 (casts are explicit)"
    with pytest.raises(nr.DTypeError) as e:
        nr.clipped_policy_loss(b16, b16, b16, None, clip)  # r = exp(logp − old) is f32
    assert msg(e) == "mul: f32 and bf16 (casts are explicit)"
    with pytest.raises(nr.DTypeError) as e:
        nr.kl_estimate(f32, h16, nr.KlEstimator.K3)
    assert msg(e) == "sub: f16 and f32 (casts are explicit)"
    with pytest.raises(nr.DTypeError) as e:
        nr.kl_estimate_backward(b16, f32, nr.KlEstimator.K1)
    assert msg(e) == "sub: f32 and bf16 (casts are explicit)"
    with pytest.raises(ValueError, match="a float tensor"):
        nr.policy_gradient_loss(f32, f32, Stub((2, 3, 4), "u8"))
    with pytest.raises(AssertionError, match="rl: mask shape"):
        nr.kl_estimate(f32, f32, nr.KlEstimator.K1, None, Stub((2, 3, 5), "f32"))
    for call in (lambda: nr.policy_gradient_loss(b16, b16, h16),
                 lambda: nr.clipped_policy_loss(h16, h16, f32, b16, clip),
                 lambda: nr.clip_fraction(b16, b16, h16, None, clip),
                 lambda: nr.kl_estimate(h16, h16, nr.KlEstimator.K2, None, b16)):
        with pytest.raises((AssertionError, nr.HipUnavailable)):  # past the dtype checks, at the device
            call()


def test_per_row_arguments_are_checked_before_any_launch():
    """Uniforms, tokens, upstream gradients and saved statistics are read as rows of f64, i32 or
    f32 by the kernels: a wrong dtype or count is refused before any device call."""
    x = Stub((2, 3, 50), "f32")
    with pytest.raises(ValueError, match=r"uniforms: dtype f32 \(f64\)"):
        nr.sample_logp(x, 0.7, None, None, uniforms=Stub((6,), "f32"))
    with pytest.raises(ValueError, match="uniforms: 5 values for 6 rows"):
        nr.sample_logp(x, 0.7, None, None, uniforms=Stub((5,), "f64"))
    with pytest.raises(ValueError, match=r"tokens: dtype u8 \(i32\)"):
        nr.token_log_probs(x, Stub((2, 3), "u8"))
    st = nr.RowStats(Stub((2, 3), "f32"), Stub((2, 3), "f32"))
    with pytest.raises(ValueError, match="g_logp: 5 values for 6 rows"):
        nr.score_grad(x, None, Stub((2, 3), "i32"), st, g_logp=Stub((5,), "f32"))
    with pytest.raises(ValueError, match=r"g_entropy: a float tensor"):
        nr.score_grad(x, None, None, st, entropy=Stub((2, 3), "f32"), g_entropy=Stub((2, 3), "i32"))
    with pytest.raises(ValueError, match="lse_rest: 4 values for 6 rows"):
        nr.score_grad(x, None, None, nr.RowStats(Stub((2, 3), "f32"), Stub((4,), "f32")),
                      entropy=Stub((2, 3), "f32"), g_entropy=Stub((2, 3), "f32"))
