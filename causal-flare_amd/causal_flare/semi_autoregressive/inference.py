"""Semi-autoregressive cached prefill/decode.

The reference ships these entry points as stubs that raise
``NotImplementedError`` (``causal_flare/semi_autoregressive/inference.py:5-36``);
this build keeps the same names and behaviour.
"""
import torch.autograd as autograd


class SemiAutoRegressivePrefillFLARE(autograd.Function):
    @staticmethod
    def forward(ctx, Q, K, V, state=None, scale=None, attention_mask=None, Q_dec=None, K_dec=None):
        raise NotImplementedError("SemiAutoRegressivePrefillFLARE is not implemented yet.")

    @staticmethod
    def backward(ctx, dY, dState=None):
        raise NotImplementedError("SemiAutoRegressivePrefillFLARE backward is not implemented yet.")


class SemiAutoRegressiveDecodeFLARE(autograd.Function):
    @staticmethod
    def forward(ctx, Q, K, V, state=None, scale=None, Q_dec=None, K_dec=None):
        raise NotImplementedError("SemiAutoRegressiveDecodeFLARE is not implemented yet.")

    @staticmethod
    def backward(ctx, dY, dState=None):
        raise NotImplementedError("SemiAutoRegressiveDecodeFLARE backward is not implemented yet.")


def flare_semi_autoregressive_prefill_trition(Q, K, V, *, state=None, scale=None, attention_mask=None, Q_dec=None,
                                              K_dec=None):
    raise NotImplementedError("flare_semi_autoregressive_prefill_trition is not implemented yet.")


def flare_semi_autoregressive_decode_trition(Q, K, V, *, state=None, scale=None, Q_dec=None, K_dec=None):
    raise NotImplementedError("flare_semi_autoregressive_decode_trition is not implemented yet.")
