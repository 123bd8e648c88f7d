"""Learning-rate schedules (reference `src/lr.ts`). A schedule is a number or a dict
with `kind` in linear / cosineAnnealing / warmup / staircase / multiStep and an optional
`startStep` (lr.ts:19-25); `resolve_lr` restates lr.ts:69-105, `rebase_lr` lr.ts:108-112.
The same arithmetic is implemented in the C++ runtime (`tg_lr.cpp`), which is what a
training step uses; this copy serves the Python host API and its tests."""
from __future__ import annotations

import math
from typing import Union

LR = Union[float, int, dict]


def linear(peak, final, steps, startStep=None) -> dict:
    return _mk('linear', peak=peak, final=final, steps=steps, startStep=startStep)


def cosine_annealing(peak, final, steps, startStep=None) -> dict:
    return _mk('cosineAnnealing', peak=peak, final=final, steps=steps, startStep=startStep)


def warmup(peak, steps, after, startStep=None) -> dict:
    return _mk('warmup', peak=peak, steps=steps, after=after, startStep=startStep)


def staircase(peak, every, gamma, startStep=None) -> dict:
    return _mk('staircase', peak=peak, every=every, gamma=gamma, startStep=startStep)


def multi_step(peak, milestones, gamma, startStep=None) -> dict:
    return _mk('multiStep', peak=peak, milestones=list(milestones), gamma=gamma, startStep=startStep)


def _mk(kind, **kw) -> dict:
    d = {'kind': kind}
    d.update({k: v for k, v in kw.items() if v is not None})
    return d


def _intrinsic(start_step, step) -> float:
    return max(1, step - (start_step or 0))


def resolve_lr(schedule: LR, step: float) -> float:
    if isinstance(schedule, (int, float)):
        return schedule
    k = schedule['kind']
    s = _intrinsic(schedule.get('startStep'), step)
    if k == 'linear':
        f = min(s / schedule['steps'], 1)
        return schedule['peak'] + (schedule['final'] - schedule['peak']) * f
    if k == 'cosineAnnealing':
        f = min(s / schedule['steps'], 1)
        return schedule['final'] + 0.5 * (schedule['peak'] - schedule['final']) * (1 + math.cos(math.pi * f))
    if k == 'warmup':
        if s <= schedule['steps']:
            return schedule['peak'] * (s / schedule['steps'])
        return resolve_lr(schedule['after'], s - schedule['steps'])
    if k == 'staircase':
        kk = math.floor((s - 1) / schedule['every'])
        return schedule['peak'] * math.pow(schedule['gamma'], kk)
    if k == 'multiStep':
        kk = sum(1 for m in schedule['milestones'] if s >= m)
        return schedule['peak'] * math.pow(schedule['gamma'], kk)
    raise ValueError(f'unknown lr schedule kind {k!r}')


def rebase_lr(schedule: LR, base_step: int) -> LR:
    if isinstance(schedule, (int, float)):
        return schedule
    if schedule.get('startStep') is not None:
        return schedule
    out = dict(schedule)
    out['startStep'] = base_step - 1
    return out


def is_lr_dynamic(schedule: LR) -> bool:
    return not isinstance(schedule, (int, float))
