"""Scenes to and from JSON (a composed task saved once and loaded where its sources are absent).

The document holds the scene's bodies (joints, geoms, sites), actuators, options, the controller
configuration, sensors and the per-world initial state, with floats written by ``repr`` so that a
round trip is exact.
"""
from __future__ import annotations

import dataclasses
import json

import numpy as np

from . import scene as S

SCHEMA = 'libero-hip-scene-v1'


def _plain(x):
    if isinstance(x, np.ndarray):
        return x.tolist()
    if isinstance(x, (np.floating, np.integer)):
        return x.item()
    if isinstance(x, (list, tuple)):
        return [_plain(v) for v in x]
    if isinstance(x, dict):
        return {k: _plain(v) for k, v in x.items()}
    return x


def _record(obj):
    return {f.name: _plain(getattr(obj, f.name)) for f in dataclasses.fields(obj)}


def to_dict(sc: S.Scene):
    bodies = []
    for b in sc.bodies:
        d = _record(b)
        d['joints'] = [_record(j) for j in b.joints]
        d['geoms'] = [_record(g) for g in b.geoms]
        d['sites'] = [_record(s) for s in b.sites]
        bodies.append(d)
    return dict(schema=SCHEMA, name=sc.name, nworld=sc.nworld, substeps=sc.substeps, seed=sc.seed,
                bodies=bodies, actuators=[_record(a) for a in sc.actuators], options=_record(sc.options),
                osc=_plain(sc.osc), sensors=[_record(s) for s in sc.sensors],
                init_qpos=_plain(sc.init_qpos), init_qvel=_plain(sc.init_qvel),
                body_active=None if sc.body_active is None else _plain(sc.body_active))


def _tuples(cls, d):
    """Dataclass from a dict, lists turned back into tuples where the field default is a tuple."""
    kw = {}
    for f in dataclasses.fields(cls):
        if f.name not in d:
            continue
        v = d[f.name]
        if isinstance(v, list) and isinstance(f.default, tuple):
            v = tuple(v)
        kw[f.name] = v
    return cls(**kw)


def from_dict(d):
    if d.get('schema') != SCHEMA:
        raise ValueError('not a %s document' % SCHEMA)
    bodies = []
    for bd in d['bodies']:
        b = _tuples(S.Body, {k: v for k, v in bd.items() if k not in ('joints', 'geoms', 'sites')})
        b.joints = [_tuples(S.Joint, j) for j in bd['joints']]
        b.geoms = []
        for g in bd['geoms']:
            geom = _tuples(S.Geom, {k: v for k, v in g.items() if k != 'vertices'})
            if g.get('vertices') is not None:
                geom.vertices = np.asarray(g['vertices'], float)
            b.geoms.append(geom)
        b.sites = [_tuples(S.Site, s) for s in bd['sites']]
        bodies.append(b)
    osc = dict(d['osc'])
    for k in ('kp', 'kd', 'q0'):
        osc[k] = np.asarray(osc[k], float)
    return S.Scene(name=d['name'], bodies=bodies, actuators=[_tuples(S.Actuator, a) for a in d['actuators']],
                   options=_tuples(S.Options, d['options']), nworld=d['nworld'], substeps=d['substeps'],
                   osc=osc, init_qpos=np.asarray(d['init_qpos'], float), init_qvel=np.asarray(d['init_qvel'], float),
                   body_active=None if d['body_active'] is None else np.asarray(d['body_active'], np.int32),
                   seed=d['seed'], sensors=[_tuples(S.Sensor, s) for s in d['sensors']])


def save(sc, path):
    with open(path, 'w') as f:
        json.dump(to_dict(sc), f, separators=(',', ':'))


def load(path):
    with open(path) as f:
        return from_dict(json.load(f))
