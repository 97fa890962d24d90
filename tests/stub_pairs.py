"""Pure-torch autograd pairs with the reference's signatures — CPU stand-ins used
only to test the binding and verification wiring (no GPU needed). SABOTAGE
switches plant mistakes so the gate can be shown to name them."""

import torch

SABOTAGE = {"wrong_dweight": False, "wrong_forward": False, "scalar_saved": False}


def rmsnorm_forward_with_saved(x, weight, eps=1e-5):
    x32 = x.float()
    rstd = torch.rsqrt((x32 * x32).mean(-1, keepdim=True) + eps)
    y = (x32 * rstd * weight.float()).to(x.dtype)
    if SABOTAGE["wrong_forward"]:
        y = y * 1.5
    saved = (x, weight, rstd)
    if SABOTAGE["scalar_saved"]:
        saved = saved + ("block=128", 7)
    return y, saved


def rmsnorm_backward_from_saved(dy, saved, eps=1e-5):
    x, weight, rstd = saved[:3]
    xh = x.float() * rstd
    g = dy.float() * weight.float()
    dx = (g - xh * (g * xh).mean(-1, keepdim=True)) * rstd
    dw = (dy.float() * xh).sum(0)
    if SABOTAGE["wrong_dweight"]:
        dw = dw + 1.0
    return dx.to(x.dtype), dw.to(weight.dtype)


def softmax_forward_with_saved(x):
    y = torch.softmax(x.float(), -1).to(x.dtype)
    return y, (y,)


def softmax_backward_from_saved(dy, saved):
    (y,) = saved
    y32 = y.float()
    return (y32 * (dy.float() - (dy.float() * y32).sum(-1, keepdim=True))).to(y.dtype)
