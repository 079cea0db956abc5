"""Sampler patches of the generation loop — drop-in for kernels/fast_sampler.py.

  install(parity=False) / uninstall() / stats()      (kernels/fast_sampler.py:113-143)

Patched (transformers generation_diffusion_gemma):
- EntropyBoundSampler.accept_canvas and StableAndConfidentStoppingCriteria.__call__
  compute the same token entropy of the same logits tensor once per step:
  the first result is cached under (data_ptr, _version) and reused
  (kernels/fast_sampler.py:24-63). Bitwise tier (parity=False): the entropy is
  the stock Categorical chain, so generation is unchanged bit for bit.
- parity=True: DiffusionGemmaGenerationMixin._denoising_step samples with the
  Gumbel-max kernel instead of softmax + multinomial + argmax
  (kernels/fast_sampler.py:68-110), and the entropy is the one-pass kernel.
  Here one call (sample_step) yields the sample, the argmax and the entropy
  from a single read of the logits, and the entropy is cached for the sampler
  and the stopping criterion, so the logits are read once per step (the
  reference reads them twice). The seed derivation is the reference's, so a
  seeded run draws the same tokens.
"""
from __future__ import annotations

import torch

_STATE: dict = {}
_ORIG: dict = {}
_PARITY = {"on": False}


def _gen():
    from transformers.models.diffusion_gemma import generation_diffusion_gemma as G
    return G


def _entropy(logits):
    """Tier dispatch: bitwise tier = stock Categorical chain; parity tier = the one-pass kernel."""
    if _PARITY["on"]:
        from .fused_sampler_ops import fused_entropy
        return fused_entropy(logits)
    return torch.distributions.Categorical(logits=logits).entropy()


def _step_entropy(logits):
    """The sampler's entropy, first of the step: computed and cached (a key
    can repeat across steps when a new logits tensor reuses freed memory, so
    an older entry is never read here), unless the parity step has just
    cached it for this very tensor."""
    key = (logits.data_ptr(), logits._version)
    if _STATE.pop("fresh", None) == key and _STATE.get("key") == key:
        return _STATE["entropy"]
    h = _entropy(logits)
    _STATE["key"] = key
    _STATE["entropy"] = h
    return h


def _cached_entropy(logits):
    """The stopping criterion's entropy: the sampler's when the tensor is byte-identical."""
    if _STATE.get("key") == (logits.data_ptr(), logits._version):
        _STATE["hits"] = _STATE.get("hits", 0) + 1
        return _STATE["entropy"]
    _STATE["misses"] = _STATE.get("misses", 0) + 1
    return _entropy(logits)


def _accept_canvas(self, current_canvas, denoiser_canvas, logits, cur_step):
    """EntropyBoundSampler.accept_canvas (TF generation_diffusion_gemma.py:406-450)
    with the step's entropy cached for the stopping criterion."""
    token_entropy = _step_entropy(logits)
    sorted_token_entropy, sorted_indices = torch.sort(token_entropy, dim=-1, descending=False)
    cumulative_entropy = torch.cumsum(sorted_token_entropy, dim=-1)
    sorted_selection_mask = cumulative_entropy - sorted_token_entropy <= self.entropy_bound
    self.accepted_token_mask = torch.scatter(input=torch.zeros_like(sorted_selection_mask), dim=-1,
                                             index=sorted_indices, src=sorted_selection_mask)
    return torch.where(self.accepted_token_mask, denoiser_canvas, current_canvas)


def _stop_call(self, argmax_canvas, logits, **kwargs):
    """StableAndConfidentStoppingCriteria.__call__ (TF generation_diffusion_gemma.py:503-536):
    the stability part unchanged, the confidence part on the cached entropy."""
    if self.stability_threshold == 0:
        stable = torch.ones((logits.shape[0]), device=logits.device, dtype=torch.bool)
    else:
        if self.argmax_canvas_history is None:
            self.argmax_canvas_history = torch.full(
                (self.stability_threshold, argmax_canvas.shape[0], argmax_canvas.shape[1]), -1,
                dtype=argmax_canvas.dtype, device=argmax_canvas.device)
        stable = (self.argmax_canvas_history == argmax_canvas[None, :, :]).all(dim=-1).all(dim=0)
        self.argmax_canvas_history = torch.roll(self.argmax_canvas_history, shifts=-1, dims=0)
        self.argmax_canvas_history[-1] = argmax_canvas
    token_entropy = _cached_entropy(logits)
    confident = torch.mean(token_entropy, dim=-1) < self.confidence_threshold
    return stable & confident


def step_seed(step: int) -> int:
    """The Gumbel seed of a denoising step: one draw of the CPU torch generator
    (seeded per question, so runs reproduce) mixed with the step index
    (kernels/fast_sampler.py:92)."""
    return (int(torch.randint(0, 2 ** 31 - 1, (1,)).item()) ^ (int(step) * 0x9E3779B1)) & 0x7FFFFFFF


def _denoising_step_parity(self, decoder_forward, current_canvas, argmax_canvas, input_ids, decoder_position_ids,
                           self_conditioning_logits, mask_mapping, past_key_values, finished_denoising, cur_step,
                           sampler, logits_processor, diffusion_stopping_criteria, **model_kwargs):
    """DiffusionGemmaGenerationMixin._denoising_step (TF generation_diffusion_gemma.py:1003-1071)
    with its sampling block (softmax, multinomial, argmax) replaced by one
    sample_step call whose entropy feeds the per-step cache."""
    from .fused_sampler_ops import sample_step
    step_int = int(cur_step)
    cur_step = torch.tensor(cur_step, device=current_canvas.device, dtype=torch.int32)
    torch.compiler.cudagraph_mark_step_begin()
    decoder_outputs = decoder_forward(decoder_input_ids=current_canvas, self_conditioning_logits=self_conditioning_logits,
                                      decoder_attention_mask=mask_mapping, past_key_values=past_key_values,
                                      decoder_position_ids=decoder_position_ids, **model_kwargs)
    processed_logits = logits_processor(input_ids, decoder_outputs.logits, cur_step=cur_step)
    batch_size, canvas_length = current_canvas.shape
    samp, amax, token_entropy = sample_step(processed_logits, step_seed(step_int))
    key = (processed_logits.data_ptr(), processed_logits._version)
    _STATE["key"] = key
    _STATE["fresh"] = key
    _STATE["entropy"] = token_entropy
    denoiser_canvas = samp.view(batch_size, canvas_length)
    new_argmax_canvas = amax.view(batch_size, canvas_length)
    accepted_canvas = sampler.accept_canvas(current_canvas, denoiser_canvas, processed_logits, cur_step).clone()
    new_current_canvas = sampler.renoise_canvas(accepted_canvas, cur_step).clone()
    if diffusion_stopping_criteria is not None:
        if finished_denoising.any():
            new_argmax_canvas = torch.where(finished_denoising[:, None], argmax_canvas, new_argmax_canvas)
            new_current_canvas = torch.where(finished_denoising[:, None], current_canvas, new_current_canvas)
            processed_logits = torch.where(finished_denoising[:, None, None], self_conditioning_logits,
                                           processed_logits)
        finished_denoising |= diffusion_stopping_criteria(new_argmax_canvas, processed_logits)
    embeddings_dtype = self.model.decoder.embed_tokens.weight.dtype
    self_conditioning_logits = processed_logits.to(embeddings_dtype)
    return new_current_canvas, new_argmax_canvas, self_conditioning_logits, finished_denoising


def install(parity: bool = False) -> None:
    """Patch the generation loop (kernels/fast_sampler.py:113-129). Installing
    again with the other tier raises."""
    if _ORIG:
        if bool(parity) != _PARITY["on"]:
            raise RuntimeError(f"fast_sampler already installed with parity={_PARITY['on']}; "
                               f"call uninstall() before install(parity={bool(parity)})")
        return
    G = _gen()
    _PARITY["on"] = bool(parity)
    _ORIG["accept"] = G.EntropyBoundSampler.accept_canvas
    _ORIG["stop"] = G.StableAndConfidentStoppingCriteria.__call__
    G.EntropyBoundSampler.accept_canvas = _accept_canvas
    G.StableAndConfidentStoppingCriteria.__call__ = _stop_call
    if parity:
        _ORIG["step"] = G.DiffusionGemmaGenerationMixin._denoising_step
        G.DiffusionGemmaGenerationMixin._denoising_step = _denoising_step_parity
    _STATE.clear()


def uninstall() -> None:
    if not _ORIG:
        return
    G = _gen()
    G.EntropyBoundSampler.accept_canvas = _ORIG.pop("accept")
    G.StableAndConfidentStoppingCriteria.__call__ = _ORIG.pop("stop")
    if "step" in _ORIG:
        G.DiffusionGemmaGenerationMixin._denoising_step = _ORIG.pop("step")
    _PARITY["on"] = False


def stats() -> dict:
    return {k: _STATE.get(k, 0) for k in ("hits", "misses")}
