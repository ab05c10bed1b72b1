"""``HipOptimizedBackend`` at the reference's plug-in point, without a GPU: construction (the
chunk default and the aliased-state load hook of ``_optimized.py:48-51``), the settings under which
the reference's backend declines a parameter (nothing changed, no generator touched), the
parameters the kernels do not take going to the reference's own backend, and the step loop of
``adamw.py:497-502`` driving it.  The stepping itself is a GPU test (test_gpu_backend.py)."""

import pytest
import torch

from adamw4bit_amd.adamw import _FALLBACK_KEY, QuantizedAdamW
from adamw4bit_amd.backend import HipOptimizedBackend
from adamw4bit_amd.quantization import QuantState

from tests.reference_like import ReferenceLikeOptimizer


class StubReferenceBackend:
    """Stands in for the reference's OptimizedBackend: records what it is offered."""

    def __init__(self, answer: bool):
        self.answer = answer
        self.calls = []

    def try_step_parameter(self, optimizer, parameter, group):
        self.calls.append(parameter)
        return self.answer


def make(params, answer=False, **kw):
    stub = StubReferenceBackend(answer)
    opt = ReferenceLikeOptimizer(params, backend=HipOptimizedBackend, reference_backend=stub,
                                 quant_state_type=QuantState, **kw)
    return opt, stub


def with_grad(*shape, dtype=torch.float32):
    p = torch.nn.Parameter(torch.zeros(shape, dtype=dtype))
    p.grad = torch.ones_like(p)
    return p


def test_construction_sets_the_chunk_default_and_the_load_hook():
    opt, _ = make([with_grad(4096)])
    assert opt.param_groups[0]["max_chunk_numel"] == 1 << 19
    assert QuantizedAdamW._after_load in opt._optimizer_load_state_dict_post_hooks.values()


@pytest.mark.parametrize("setting", ["update_sign_clip", "update_norm_clip", "record_update_direction_every",
                                     "record_preconditioner_every", "record_preconditioner_steps", "telemetry"])
def test_declining_settings_change_nothing_and_draw_nothing(setting):
    p = with_grad(64, 128)
    opt, stub = make([p])
    if setting == "telemetry":
        opt.telemetry = object()
    else:
        opt.param_groups[0][setting] = 1
    opt.step()
    assert opt.declined == [p] and stub.calls == []
    assert p not in opt.state and opt._quant_generators == {"m1": {}, "m2": {}}
    assert torch.equal(p.detach(), torch.zeros_like(p))


@pytest.mark.parametrize("answer", [True, False])
def test_parameters_the_kernels_do_not_take_go_to_the_reference_backend(answer):
    """CPU parameters (and complex ones) are the reference backend's: its answer is the answer."""
    ps = [with_grad(64, 128), with_grad(4096, dtype=torch.complex64)]
    opt, stub = make(ps, answer=answer)
    opt.step()
    assert stub.calls == ps
    assert opt.declined == ([] if answer else ps)


def test_the_backend_belongs_to_its_optimizer():
    opt, _ = make([with_grad(4096)])
    other, _ = make([with_grad(4096)])
    with pytest.raises(ValueError, match="another optimizer"):
        opt._optimized_backend.try_step_parameter(other, other.param_groups[0]["params"][0], other.param_groups[0])


def test_checkpoint_load_restores_codes_before_the_aliasing_hook():
    """torch's load casts a parameter's state tensors to its dtype; the reference's loader (and the
    stand-in) puts the uint8 codes and fp32 scales back in a post-hook that runs first, so the
    backend's aliased-state hook sees the restored state and marks nothing."""
    p = torch.nn.Parameter(torch.zeros(64, 128, dtype=torch.bfloat16))
    opt, _ = make([p])
    codes = torch.arange(64 * 128 // 2, dtype=torch.uint8)
    opt.state[p].update(step=3, m1_code=codes, m2_code=codes.flip(0).clone(),
                        m1_quant_state=QuantState(torch.rand(64), shape=p.shape, dtype=torch.float32, blocksize=128,
                                                  packed=True),
                        m2_quant_state=QuantState(torch.rand(64), shape=p.shape, dtype=torch.float32, blocksize=128,
                                                  packed=True))
    saved = opt.state_dict()
    seen = {}
    q = torch.nn.Parameter(torch.zeros(64, 128, dtype=torch.bfloat16))
    resumed, _ = make([q])
    resumed.register_load_state_dict_post_hook(lambda o: seen.update(dtype=o.state[q]["m1_code"].dtype))
    resumed.load_state_dict(saved)
    st = resumed.state[q]
    assert seen["dtype"] == torch.uint8
    assert st["m1_code"].dtype == torch.uint8 and torch.equal(st["m1_code"], codes)
    assert isinstance(st["m2_quant_state"], QuantState) and st["m2_quant_state"].absmax.dtype == torch.float32
    assert torch.equal(st["m2_quant_state"].absmax, opt.state[p]["m2_quant_state"].absmax)
    assert _FALLBACK_KEY not in st and st["step"] == 3
