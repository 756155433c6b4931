"""CausalLM.forward with the fused lm_head + cross-entropy (reference
forge/forge/patching/kernels/fused_linear_ce.py:16-140).

In training with labels (and logits_to_keep == 0) the last hidden states are
shifted by one token and handed to forge_fused_linear_cross_entropy with the
live lm_head weight and bias, so no [B*T, V] logits tensor is formed; the
model returns loss and logits=None.  Otherwise (eval, no labels, a
logits_to_keep slice) it computes logits through lm_head and, with labels,
the model's own loss_function - the unpatched behaviour.
"""
from __future__ import annotations


def _unpack_cross_entropy_result(result):
    """(loss, token_accuracy, predicted_tokens) from the fused entry's result:
    an object with .loss, a tuple (loss, z_loss, accuracy, predicted), or a
    bare loss (fused_linear_ce.py:5-13)."""
    if hasattr(result, "loss"):
        return result.loss, getattr(result, "token_accuracy", None), getattr(result, "predicted_tokens", None)
    if isinstance(result, tuple):
        return (result[0], result[2] if len(result) > 2 else None, result[3] if len(result) > 3 else None)
    return result, None, None


def make_fused_linear_ce_forward(module, config):
    """Factory for a `*ForCausalLM` module; the forward takes HF's CausalLM
    arguments plus the loss keywords the reference pops from kwargs
    (shift_labels, skip_logits, num_items_in_batch, ignore_index,
    label_smoothing, final_logit_softcapping, accum_dtype,
    return_token_accuracy, return_predicted_tokens)."""
    from transformers.modeling_outputs import CausalLMOutputWithPast

    from forge.kernels.cross_entropy import forge_fused_linear_cross_entropy

    loss_keys = {"shift_labels": None, "skip_logits": None, "num_items_in_batch": None, "ignore_index": -100,
                 "label_smoothing": 0.0, "final_logit_softcapping": None, "accum_dtype": None,
                 "return_token_accuracy": False, "return_predicted_tokens": False}

    def forward(input_ids=None, attention_mask=None, position_ids=None, past_key_values=None, inputs_embeds=None,
                labels=None, use_cache=None, output_attentions=None, output_hidden_states=None, cache_position=None,
                logits_to_keep=0, **kwargs):
        cfg = module.config
        return_dict = kwargs.pop("return_dict", None)
        if return_dict is None:
            return_dict = getattr(cfg, "use_return_dict", True)
        opt = {k: kwargs.pop(k, d) for k, d in loss_keys.items()}
        shift_labels = opt["shift_labels"]
        if output_attentions is None:
            output_attentions = getattr(cfg, "output_attentions", False)
        if output_hidden_states is None:
            output_hidden_states = getattr(cfg, "output_hidden_states", False)

        outputs = module.model(input_ids=input_ids, attention_mask=attention_mask, position_ids=position_ids,
                               past_key_values=past_key_values, inputs_embeds=inputs_embeds, use_cache=use_cache,
                               output_attentions=output_attentions, output_hidden_states=output_hidden_states,
                               cache_position=cache_position, **kwargs)
        hidden = outputs.last_hidden_state if hasattr(outputs, "last_hidden_state") else outputs[0]

        has_labels = labels is not None or shift_labels is not None
        skip_logits = opt["skip_logits"]
        if skip_logits and not has_labels:
            raise ValueError("skip_logits is True, but labels and shift_labels are None")
        if skip_logits is None:
            skip_logits = module.training and has_labels

        loss = logits = token_accuracy = predicted_tokens = None
        if skip_logits and isinstance(logits_to_keep, int) and logits_to_keep == 0 and has_labels:
            if shift_labels is None:  # predict token t+1 from position t
                h = hidden[..., :-1, :].contiguous()
                shift_labels = labels[..., 1:].contiguous()
            else:
                h = hidden
            h = h.view(-1, cfg.hidden_size)
            reduction = "sum" if opt["num_items_in_batch"] is not None else "mean"
            result = forge_fused_linear_cross_entropy(
                h, module.lm_head.weight, shift_labels.view(-1).to(h.device),
                bias=getattr(module.lm_head, "bias", None), ignore_index=opt["ignore_index"],
                label_smoothing=opt["label_smoothing"], reduction=reduction,
                softcap=opt["final_logit_softcapping"], accum_dtype=opt["accum_dtype"],
                return_token_accuracy=opt["return_token_accuracy"],
                return_predicted_tokens=opt["return_predicted_tokens"])
            loss, token_accuracy, predicted_tokens = _unpack_cross_entropy_result(result)
            if opt["num_items_in_batch"] is not None:
                loss = loss / opt["num_items_in_batch"]
        else:
            keep = slice(-logits_to_keep, None) if isinstance(logits_to_keep, int) else logits_to_keep
            logits = module.lm_head(hidden[:, keep, :])
            if has_labels:
                loss = module.loss_function(logits=logits, labels=labels, shift_labels=shift_labels,
                                            vocab_size=cfg.vocab_size,
                                            num_items_in_batch=opt["num_items_in_batch"],
                                            ignore_index=opt["ignore_index"],
                                            label_smoothing=opt["label_smoothing"], **kwargs)

        if not return_dict:
            out = (logits,) + tuple(outputs[1:])
            if loss is not None:
                out = (loss,) + out
            return out + tuple(t for t in (token_accuracy, predicted_tokens) if t is not None)

        res = CausalLMOutputWithPast(loss=loss, logits=logits, past_key_values=outputs.past_key_values,
                                     hidden_states=outputs.hidden_states, attentions=outputs.attentions)
        if token_accuracy is not None:
            res.token_accuracy = token_accuracy
        if predicted_tokens is not None:
            res.predicted_tokens = predicted_tokens
        return res

    return forward
