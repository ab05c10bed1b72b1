"""A stand-in with the interface the reference's ``QuantizedAdamW`` offers its optimized backend
(``adamw.py``: constructor defaults and group keys, ``_m1_scheme_for``, ``_effective_scheme``,
``_quant_generator`` and its seeds, ``telemetry``, the ``_last_*`` records, and the ``step()``
loop that asks ``_optimized_backend.try_step_parameter`` first, ``adamw.py:497-502``), written
from that interface for the tests of ``adamw4bit_amd.backend``; its own step for declined
parameters only counts them.  Test infrastructure: the reference package itself is not imported."""

from __future__ import annotations

import torch

from adamw4bit_amd.quantization import QuantState  # stands in for the reference's QuantState

MIN_QUANT_NUMEL = 4096


class ReferenceLikeOptimizer(torch.optim.Optimizer):
    QUANT_RNG_OFFSETS = {"m1": 0x1A2B3C4D, "m2": 0x5E6F7789}

    def __init__(self, params, *, lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1,
                 m1_quant_scheme="nf4", m2_quant_scheme="dyn4_upd_sr_fp32read", use_eden_m2=False,
                 quant_rng_seed=0, backend=None, **backend_kwargs):
        defaults = dict(lr=lr, betas=betas, eps=eps, weight_decay=weight_decay, block_size=None,
                        use_eden_m2=use_eden_m2, m1_quant_scheme=m1_quant_scheme, m2_quant_scheme=m2_quant_scheme,
                        update_sign_clip=None, update_norm_clip=None, record_update_direction_every=None,
                        record_preconditioner_every=None, record_preconditioner_steps=None)
        super().__init__(params, defaults)
        self._quant_rng_seed = quant_rng_seed
        self._quant_generators = {"m1": {}, "m2": {}}
        self._m1_quant_scheme_overrides = {}
        self._last_update_directions, self._last_preconditioners = {}, {}
        self._last_effective_preconditioners = {}
        self.telemetry = None
        self.declined = []  # parameters the backend declined, stepped by "the reference step"
        self._optimized = True
        self._optimized_backend = backend(self, **backend_kwargs) if backend is not None else None

    def _m1_scheme_for(self, parameter, group_scheme):
        return self._m1_quant_scheme_overrides.get(id(parameter), group_scheme)

    @staticmethod
    def _effective_scheme(p, scheme, block_size):
        # the TorchAO eligibility rule: small or unaligned tensors keep fp32 state
        if p.numel() < MIN_QUANT_NUMEL or p.numel() % block_size:
            return "fp32"
        return scheme

    def _quant_generator(self, moment, device):
        if self._quant_rng_seed is None:
            return None
        generators = self._quant_generators[moment]
        key = str(device)
        if key not in generators:
            g = torch.Generator(device=device)
            g.manual_seed((self._quant_rng_seed + self.QUANT_RNG_OFFSETS[moment]) % ((1 << 63) - 1))
            generators[key] = g
        return generators[key]

    def generator_states(self):
        return {m: {k: g.get_state() for k, g in gens.items()} for m, gens in self._quant_generators.items()}

    def set_generator_states(self, states):
        for m, gens in states.items():
            for key, state in gens.items():
                self._quant_generator(m, torch.device(key)).set_state(state)

    def state_dict(self):
        """torch's state dict with each moment's scale metadata as a plain dict (adamw.py:326-336)."""
        out = super().state_dict()
        out["state"] = {index: {k: (vars(v).copy() if isinstance(v, QuantState) else v) for k, v in st.items()}
                        for index, st in out["state"].items()}
        return out

    def load_state_dict(self, state_dict):
        """torch's load casts every tensor of a parameter's state to the parameter's dtype; as the
        reference does (adamw.py:364-425), a post-hook that runs before any other puts back the
        saved fp32 moments and uint8 codes and rebuilds the scale metadata objects."""
        def restore(_optimizer):
            for group, saved_group in zip(self.param_groups, state_dict["param_groups"]):
                for p, index in zip(group["params"], saved_group["params"]):
                    saved = state_dict["state"].get(index, {})
                    state = self.state[p]
                    for key in ("m1", "m2", "lookahead_pending_exp_avg_sq", "m2_read_preconditioner"):
                        if key in saved:
                            state[key] = saved[key].to(device=p.device, dtype=torch.float32)
                    for key in ("m1_code", "m2_code"):
                        if key in saved:
                            state[key] = saved[key].to(device=p.device, dtype=torch.uint8)
                    for key in ("m1_quant_state", "m2_quant_state"):
                        if key in saved:
                            fields = dict(saved[key])
                            fields["absmax"] = fields["absmax"].to(device=p.device, dtype=torch.float32)
                            state[key] = QuantState(**fields)

        hook = self.register_load_state_dict_post_hook(restore, prepend=True)
        try:
            return super().load_state_dict(state_dict)
        finally:
            hook.remove()

    @torch.no_grad()
    def step(self, closure=None):
        for group in self.param_groups:
            for p in group["params"]:
                if p.grad is None:
                    continue
                if self._optimized and self._optimized_backend.try_step_parameter(self, p, group):
                    continue
                self.declined.append(p)
        flush = getattr(self._optimized_backend, "flush", None)
        if flush is not None:
            flush(self)
