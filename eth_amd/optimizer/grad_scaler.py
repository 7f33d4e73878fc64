"""Loss scalers with a host-side mirror of the scale.

Same update rule as eth/runtime/megatron/optimizer/grad_scaler.py:24-122
(growth x2 after `growth_interval` clean steps, backoff after `hysteresis`
overflows, floor at `min_scale`).  The scale lives on the host as well as in
a device tensor, so the fused kernels get `inv_scale` by value and the step
never waits for the device to learn it.  `inv_scale` is the float32 of the
double reciprocal, as in the reference (`_scale.double().reciprocal().float()`).
"""

import numpy as np
import torch


class MegatronGradScaler:
    def __init__(self, initial_scale, device=None):
        if not initial_scale > 0.0:
            raise ValueError("initial_scale must be positive")
        self._host_scale = float(np.float32(initial_scale))
        self._device = device
        self._scale_tensor = None

    @property
    def host_scale(self):
        return self._host_scale

    @property
    def scale(self):
        dev = self._device if self._device is not None else ("cuda" if torch.cuda.is_available() else "cpu")
        if self._scale_tensor is None or float(self._scale_tensor_host) != self._host_scale:
            self._scale_tensor = torch.tensor([self._host_scale], dtype=torch.float32, device=dev)
            self._scale_tensor_host = self._host_scale
        return self._scale_tensor

    @property
    def inv_scale_value(self):
        return float(np.float32(1.0 / np.float64(self._host_scale)))

    @property
    def inv_scale(self):
        return torch.tensor([self.inv_scale_value], dtype=torch.float32, device=self.scale.device)

    def update(self, found_inf):
        raise NotImplementedError

    def state_dict(self):
        raise NotImplementedError

    def load_state_dict(self, state_dict):
        raise NotImplementedError


class ConstantGradScaler(MegatronGradScaler):
    def update(self, found_inf):
        pass

    def state_dict(self):
        return {}

    def load_state_dict(self, state_dict):
        pass


class DynamicGradScaler(MegatronGradScaler):
    def __init__(self, initial_scale, min_scale, growth_factor, backoff_factor, growth_interval, hysteresis, device=None):
        super().__init__(initial_scale, device)
        if not (0.0 < min_scale <= initial_scale):
            raise ValueError("min_scale must be in (0, initial_scale]")
        if not growth_factor > 1.0:
            raise ValueError("growth_factor must exceed 1")
        if not 0.0 < backoff_factor < 1.0:
            raise ValueError("backoff_factor must be in (0, 1)")
        if growth_interval <= 0 or hysteresis <= 0:
            raise ValueError("growth_interval and hysteresis must be positive")
        self.min_scale = float(np.float32(min_scale))
        self.growth_factor = float(np.float32(growth_factor))
        self.backoff_factor = float(np.float32(backoff_factor))
        self.growth_interval = growth_interval
        self.hysteresis = hysteresis
        self._growth_tracker = 0
        self._hysteresis_tracker = hysteresis

    def update(self, found_inf):
        f32 = np.float32
        if found_inf:
            self._growth_tracker = 0
            self._hysteresis_tracker -= 1
            if self._hysteresis_tracker <= 0:
                self._host_scale = float(max(f32(self._host_scale) * f32(self.backoff_factor), f32(self.min_scale)))
        else:
            self._growth_tracker += 1
            if self._growth_tracker == self.growth_interval:
                self._growth_tracker = 0
                self._hysteresis_tracker = self.hysteresis
                self._host_scale = float(f32(self._host_scale) * f32(self.growth_factor))

    def state_dict(self):
        return {
            "scale": self.scale.clone(),
            "growth_tracker": self._growth_tracker,
            "hysteresis_tracker": self._hysteresis_tracker,
        }

    def load_state_dict(self, state_dict):
        self._host_scale = float(state_dict["scale"].reshape(-1)[0].item())
        self._growth_tracker = state_dict["growth_tracker"]
        self._hysteresis_tracker = state_dict["hysteresis_tracker"]
