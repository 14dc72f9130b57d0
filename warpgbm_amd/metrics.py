"""Evaluation metrics (warpgbm/metrics.py:5-37), used by eval / early stopping.

These are plain torch expressions over device tensors: evaluation is not on
the accelerated path.
"""
import torch


def rmsle_torch(y_true, y_pred, eps=1e-7):
    """Root mean squared difference of log1p(max(v, 0) + eps) between
    targets and predictions (negative values count as 0)."""
    d = torch.log1p(y_true.clamp(min=0) + eps) - torch.log1p(y_pred.clamp(min=0) + eps)
    return d.pow(2).mean().sqrt()


def softmax(logits, dim=-1):
    """exp(x - max) / sum exp(x - max) along ``dim``."""
    e = torch.exp(logits - torch.max(logits, dim=dim, keepdim=True)[0])
    return e / torch.sum(e, dim=dim, keepdim=True)


def log_loss_torch(y_true_labels, y_pred_probs, eps=1e-15):
    """Mean negative log-likelihood of the true class, probabilities clipped to [eps, 1-eps]."""
    p = torch.clamp(y_pred_probs, eps, 1 - eps)
    n = y_true_labels.shape[0]
    return -torch.mean(torch.log(p[torch.arange(n, device=p.device), y_true_labels.long()]))


def accuracy_torch(y_true_labels, y_pred_labels):
    return (y_true_labels == y_pred_labels).float().mean()
