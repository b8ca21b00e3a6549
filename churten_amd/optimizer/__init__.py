"""Ensemble optimizers over the consolidated state (reference
src/torchstrap/optimizer/__init__.py)."""

from churten_amd.optimizer.adagrad import Adagrad, adagrad_step_
from churten_amd.optimizer.adam import Adam, adam_step_
from churten_amd.optimizer.grad_transform import GradientTransformation
from churten_amd.optimizer.sgd import SGD, sgd_step_

__all__ = ["GradientTransformation", "Adam", "SGD", "Adagrad", "adam_step_", "sgd_step_",
           "adagrad_step_"]
