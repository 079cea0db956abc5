"""Sampler patches of the diffusion generation loop: install(parity) /
uninstall() / stats(), with the tiers of kernels/fast_sampler.py:113-143.

What a denoising step of transformers' generation_diffusion_gemma does with
the logits, and what changes here:

- EntropyBoundSampler.accept_canvas and StableAndConfidentStoppingCriteria
  both compute the token entropy of the same processed-logits tensor. A
  session keeps one EntropyCache: the sampler's call computes (or receives)
  the entropy, the stopping criterion reuses it when it is handed the very
  same tensor, identified by storage pointer and version counter (the
  reference's rule, kernels/fast_sampler.py:24-63). A tensor rewritten in
  between (torch.where of a finished row, an in-place op) has another
  identity and is recomputed.
- Bitwise tier (parity=False): the entropy is torch's Categorical chain, so
  the generation is the stock one bit for bit.
- Parity tier (parity=True): the denoising step draws with the Gumbel-max
  kernel instead of softmax + multinomial, and the entropy is the one-pass
  kernel (kernels/fast_sampler.py:68-110). One sample_step call reads the
  logits once and returns the draw, the argmax and the entropy; the entropy
  goes straight into the cache, so neither the sampler nor the criterion
  reads the logits again. The draw's seed is derived as the reference does,
  so a seeded run is reproducible.

The patches are one table of (class, attribute, factory, tiers); install
applies the rows of the chosen tier and records what it replaced, uninstall
puts every recorded attribute back in reverse order.
"""
from __future__ import annotations

import dataclasses
from typing import Callable

import torch


def _generation_module():
    from transformers.models.diffusion_gemma import generation_diffusion_gemma as gen
    return gen


def _categorical_entropy(logits: torch.Tensor) -> torch.Tensor:
    return torch.distributions.Categorical(logits=logits).entropy()


def _kernel_entropy(logits: torch.Tensor) -> torch.Tensor:
    from .fused_sampler_ops import fused_entropy
    return fused_entropy(logits)


class EntropyCache:
    """The token entropy of one logits tensor per denoising step.

    first(logits): the sampler's request, the first of a step. Uses the
    entropy offered for exactly this tensor (offer()) if there is one,
    otherwise computes it; either way it becomes the cached value.
    again(logits): the stopping criterion's request. The cached value if the
    tensor is the one cached, else a fresh computation (counted as a miss).
    """

    def __init__(self, compute: Callable[[torch.Tensor], torch.Tensor]):
        self._compute = compute
        self._ident = None
        self._value = None
        self._offered = None
        self.hits = 0
        self.misses = 0

    @staticmethod
    def _identity(t: torch.Tensor):
        return t.data_ptr(), t._version

    def offer(self, logits: torch.Tensor, entropy: torch.Tensor) -> None:
        self._offered = (self._identity(logits), entropy)

    def first(self, logits: torch.Tensor) -> torch.Tensor:
        ident = self._identity(logits)
        offered, self._offered = self._offered, None
        # an offer is only good for the step that made it: a pointer can come
        # back in a later step when a new tensor reuses freed memory
        value = offered[1] if offered is not None and offered[0] == ident else self._compute(logits)
        self._ident, self._value = ident, value
        return value

    def again(self, logits: torch.Tensor) -> torch.Tensor:
        if self._ident is not None and self._ident == self._identity(logits):
            self.hits += 1
            return self._value
        self.misses += 1
        return self._compute(logits)


@dataclasses.dataclass
class _Session:
    parity: bool
    cache: EntropyCache
    replaced: list = dataclasses.field(default_factory=list)  # (class, attribute, original)


def _entropy_bound_accept(sampler, current_canvas, denoiser_canvas, token_entropy):
    """The acceptance rule of EntropyBoundSampler.accept_canvas
    (transformers generation_diffusion_gemma.py:406-450): take the tokens in
    order of increasing entropy while the entropy summed before each stays
    within the bound; accepted positions get the denoiser's token."""
    ent_sorted, order = torch.sort(token_entropy, dim=-1, descending=False)
    before = torch.cumsum(ent_sorted, dim=-1) - ent_sorted
    take_sorted = before <= sampler.entropy_bound
    sampler.accepted_token_mask = torch.scatter(input=torch.zeros_like(take_sorted), dim=-1, index=order,
                                                src=take_sorted)
    return torch.where(sampler.accepted_token_mask, denoiser_canvas, current_canvas)


def _stable_rows(criterion, argmax_canvas, batch, device):
    """The stability half of StableAndConfidentStoppingCriteria.__call__
    (transformers generation_diffusion_gemma.py:503-536): a row is stable
    when its argmax canvas equals each of the last stability_threshold ones;
    the history window then advances by one."""
    n = criterion.stability_threshold
    if n == 0:
        return torch.ones((batch,), device=device, dtype=torch.bool)
    if criterion.argmax_canvas_history is None:
        criterion.argmax_canvas_history = torch.full((n, argmax_canvas.shape[0], argmax_canvas.shape[1]), -1,
                                                     dtype=argmax_canvas.dtype, device=argmax_canvas.device)
    hist = criterion.argmax_canvas_history
    stable = (hist == argmax_canvas[None, :, :]).all(dim=-1).all(dim=0)
    criterion.argmax_canvas_history = torch.roll(hist, shifts=-1, dims=0)
    criterion.argmax_canvas_history[-1] = argmax_canvas
    return stable


def _make_accept(session: _Session):
    def accept_canvas(self, current_canvas, denoiser_canvas, logits, cur_step):
        return _entropy_bound_accept(self, current_canvas, denoiser_canvas, session.cache.first(logits))
    return accept_canvas


def _make_stop(session: _Session):
    def stopping_call(self, argmax_canvas, logits, **kwargs):
        stable = _stable_rows(self, argmax_canvas, logits.shape[0], logits.device)
        confident = torch.mean(session.cache.again(logits), dim=-1) < self.confidence_threshold
        return stable & confident
    return stopping_call


def step_seed(step: int) -> int:
    """The Gumbel seed of a denoising step: one draw of the CPU torch generator
    (seeded per question, so runs reproduce) mixed with the step index
    (kernels/fast_sampler.py:92)."""
    draw = int(torch.randint(0, 2 ** 31 - 1, (1,)).item())
    return (draw ^ (int(step) * 0x9E3779B1)) & 0x7FFFFFFF


def _make_parity_step(session: _Session):
    """DiffusionGemmaGenerationMixin._denoising_step (transformers
    generation_diffusion_gemma.py:1003-1071) in three phases: decode the
    canvas into processed logits, draw the new canvas with one sample_step
    call (its entropy offered to the cache), then the stock acceptance,
    renoising, stopping and self-conditioning."""
    from .fused_sampler_ops import sample_step

    def decode(decoder_forward, canvas, input_ids, position_ids, sc_logits, mask_mapping, past_key_values,
               logits_processor, step_t, model_kwargs):
        out = decoder_forward(decoder_input_ids=canvas, self_conditioning_logits=sc_logits,
                              decoder_attention_mask=mask_mapping, past_key_values=past_key_values,
                              decoder_position_ids=position_ids, **model_kwargs)
        return logits_processor(input_ids, out.logits, cur_step=step_t)

    def draw(logits, shape, step):
        sample, top, entropy = sample_step(logits, step_seed(step))
        session.cache.offer(logits, entropy)
        return sample.view(shape), top.view(shape)

    def denoising_step(self, decoder_forward, current_canvas, argmax_canvas, input_ids, decoder_position_ids,
                       self_conditioning_logits, mask_mapping, past_key_values, finished_denoising, cur_step,
                       sampler, logits_processor, diffusion_stopping_criteria, **model_kwargs):
        step = int(cur_step)
        step_t = torch.tensor(step, device=current_canvas.device, dtype=torch.int32)
        torch.compiler.cudagraph_mark_step_begin()
        logits = decode(decoder_forward, current_canvas, input_ids, decoder_position_ids, self_conditioning_logits,
                        mask_mapping, past_key_values, logits_processor, step_t, model_kwargs)
        drawn, top = draw(logits, current_canvas.shape, step)
        canvas = sampler.accept_canvas(current_canvas, drawn, logits, step_t).clone()
        canvas = sampler.renoise_canvas(canvas, step_t).clone()
        if diffusion_stopping_criteria is not None:
            if finished_denoising.any():
                # rows that finished earlier keep their previous results
                done = finished_denoising
                top = torch.where(done[:, None], argmax_canvas, top)
                canvas = torch.where(done[:, None], current_canvas, canvas)
                logits = torch.where(done[:, None, None], self_conditioning_logits, logits)
            finished_denoising |= diffusion_stopping_criteria(top, logits)
        next_sc = logits.to(self.model.decoder.embed_tokens.weight.dtype)
        return canvas, top, next_sc, finished_denoising

    return denoising_step


# (class in the generation module, attribute, factory of the replacement, tiers it belongs to)
_PATCHES = (
    ("EntropyBoundSampler", "accept_canvas", _make_accept, (False, True)),
    ("StableAndConfidentStoppingCriteria", "__call__", _make_stop, (False, True)),
    ("DiffusionGemmaGenerationMixin", "_denoising_step", _make_parity_step, (True,)),
)

_session: _Session | None = None
_last_stats = {"hits": 0, "misses": 0}


def install(parity: bool = False) -> None:
    """Patch the generation loop with the bitwise (parity=False) or parity
    tier. Installing again with the same tier does nothing; with the other
    tier it raises (uninstall first), so a tier is never changed silently."""
    global _session
    parity = bool(parity)
    if _session is not None:
        if _session.parity != parity:
            raise RuntimeError(f"fast_sampler is installed with parity={_session.parity}: "
                               f"uninstall() before install(parity={parity})")
        return
    gen = _generation_module()
    session = _Session(parity=parity, cache=EntropyCache(_kernel_entropy if parity else _categorical_entropy))
    for cls_name, attr, factory, tiers in _PATCHES:
        if parity not in tiers:
            continue
        cls = getattr(gen, cls_name)
        session.replaced.append((cls, attr, cls.__dict__[attr]))
        setattr(cls, attr, factory(session))
    _session = session


def uninstall() -> None:
    """Restore every attribute install() replaced (no-op when not installed)."""
    global _session
    if _session is None:
        return
    for cls, attr, original in reversed(_session.replaced):
        setattr(cls, attr, original)
    _last_stats.update(stats())
    _session = None


def installed() -> bool | None:
    """The installed tier (parity flag), or None."""
    return None if _session is None else _session.parity


def stats() -> dict:
    """Entropy cache hits and misses of the stopping criterion (the current
    session's, or the last one's after uninstall)."""
    if _session is None:
        return dict(_last_stats)
    return {"hits": _session.cache.hits, "misses": _session.cache.misses}
