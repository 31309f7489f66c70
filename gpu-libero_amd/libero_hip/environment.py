"""``HipBatchEnv``: the batch-environment façade over the world-local HIP control step.

Mirrors the public surface of ``GpuBatchEnv`` / ``CudaFP32BatchEnv``
(``gpu/host/adapters/environment/batch_env.py:94-685``, ``gpu/host/backends/cuda_fp32/environment.py:19-332``):

* ``step(actions)`` -> ``(observations, rewards, successes, infos)``, no auto-reset;
* ``reset(id=None, *, seed=None, init_states=None)``, ``set_init_state(states, id=None)``;
* ``get_sim_state()`` returns LIBERO flat ``[time | qpos | qvel]`` rows;
* ``diagnostics()``, ``work_snapshot()``, ``observation_fields()``, ``close()``, context manager;
* ``_check()`` raises ``RuntimeError`` on a fatal overflow bit or a controller error
  (``environment.py:126-140``); ITERATIONS / LS_ITERATIONS are legal exits.

Scenes come from :mod:`libero_hip.scene`.  Task predicates are outside this backend; its
boundary to them is ``_snapshot(names)`` (``gpu/host/backends/cuda_fp32/environment.py:215-254``):
one coherent read of the shaped state fields and of each world's contact geom pairs, which a
caller-supplied ``predicates(snapshot, ids) -> (rewards, successes)`` evaluates after every step
and reset (without one, rewards are 0 and successes False).  One control step is one kernel launch of
``substeps`` substeps that also samples the observation plan after every substep
(:mod:`libero_hip.observations`, the reference's graph of substeps and samples,
``gpu/host/backends/cuda_fp32/runtime.py:47-56``), optionally replayed from a captured HIP graph.
Observations are packed on the host from the device's observed values only (one copy of
``nworld x plan width`` floats per step).
"""
from __future__ import annotations

from threading import RLock

import numpy as np

from . import scene as S
from .model import Model
from . import native
from .observations import DeviceObservations, default_plan
from .selection import precision_bits, resolve_engine
from . import layout

FATAL = ~((1 << 9) | (1 << 10))

# the fields the reference's predicate boundary reads by default
# (gpu/host/adapters/observations/boundary.py:13 GOAL_FIELDS)
GOAL_FIELDS = ('qpos', 'body_xpos', 'body_xquat', 'site_xpos', 'site_xmat', 'contact', 'ncon')


class HipBatchEnv:
    physics_backend = 'gpu'
    physics_engine = 'hip_mi355x'
    is_async = False

    def __init__(self, scene='c2', num_envs=None, *, init_states=None, seed=0, scene_seed=0,
                 device='cuda:0', precision='fp32', physics_engine='hip_mi355x', graph=True,
                 substeps=25, debug=False, observation_plan=None, predicates=None, predicate_fields=GOAL_FIELDS,
                 **options):
        import torch
        resolve_engine(physics_engine, precision)
        fp64 = precision_bits(precision) == 64
        if options:
            raise ValueError('Unknown hip_mi355x options: ' + str(sorted(options)))
        if not str(device).startswith('cuda'):
            raise ValueError('A GPU device is required')
        if not torch.cuda.is_available():
            raise RuntimeError('hip_mi355x requires a ROCm GPU')
        self._lock = RLock()
        self._closed = self._failed = False
        self._predicates = predicates
        self._predicate_fields = tuple(predicate_fields)
        self.device = torch.device(device)
        self.precision = 'fp64' if fp64 else 'fp32'
        self._route = native.FLAG_FP64 if fp64 else 0   # launch flag of the precision route
        self.debug = debug
        sc = scene if isinstance(scene, S.Scene) else S.make_scene(scene, num_envs, seed=scene_seed,
                                                                   substeps=substeps)
        self.scene = sc
        self.model = Model(sc)
        self.num_envs = self.env_num = sc.nworld
        self.substeps = sc.substeps
        self.action_dim = 7
        self.seed(seed)
        native.load()
        with torch.cuda.device(self.device):
            self.stream = torch.cuda.Stream(self.device)
            self.dmodel = native.DeviceModel(self.model, self.device)
            if fp64 and self.dmodel.lds_bytes_fp64() > layout.LDS_BUDGET:
                raise ValueError('precision="fp64" keeps a world in LDS: %d bytes per world exceed the %d of a '
                                 'workgroup' % (self.dmodel.lds_bytes_fp64(), layout.LDS_BUDGET))
            self.data = native.DeviceData(self.dmodel, self.num_envs, self.device)
            d = self.data
            osc = sc.osc
            d['osc_gains'].copy_(torch.from_numpy(np.tile(np.r_[osc['kp'], osc['kd']], (self.num_envs, 1))))
            d['osc_q0'].copy_(torch.from_numpy(np.tile(np.asarray(osc['q0'], float), (self.num_envs, 1))))
            if self.model.body_active is not None:
                d['body_active'].copy_(torch.from_numpy(self.model.body_active))
            else:
                d['body_active'].fill_(1)
            self._actions_host = torch.zeros((self.num_envs, 7), dtype=torch.float64).pin_memory()
            plan = default_plan(self.model) if observation_plan is None else observation_plan
            self.observer = DeviceObservations(plan, self.model, self.num_envs, self.device)
        self.initial_states = self.model.initial_state() if init_states is None else np.asarray(init_states)
        self._graph = None
        self._use_graph = graph
        self.reset()

    # ------------------------------------------------------------------ helpers
    def seed(self, seed=None):
        self._rng = np.random.default_rng(seed)
        return [seed]

    def _open(self):
        if self._closed:
            raise RuntimeError('environment is closed')
        if self._failed:
            raise RuntimeError('environment failed; reset is not possible after a fatal error')

    def _ids(self, id):
        if id is None:
            return list(range(self.num_envs))
        ids = [int(i) for i in np.atleast_1d(id)]
        if any(i < 0 or i >= self.num_envs for i in ids) or len(set(ids)) != len(ids):
            raise ValueError('invalid world ids')
        return ids

    def _check(self):
        self.stream.synchronize()
        overflow = self.data['overflow'].cpu().numpy()[:, 0]
        errors = self.data['osc_error'].cpu().numpy()[:, 0]
        if np.any(overflow & FATAL) or np.any(errors):
            self._failed = True
            raise RuntimeError(dict(overflow=overflow.tolist(), controller_error=errors.tolist()))

    # ------------------------------------------------------------------ state
    def _restore(self, rows, ids, *, reset):
        import torch
        m = self.model
        rows = np.asarray(rows, np.float64).reshape(len(ids), 1 + m.nq + m.nv)
        idx = torch.as_tensor(ids, device=self.device, dtype=torch.long)
        d = self.data
        with torch.cuda.stream(self.stream):
            d['time'][idx] = torch.as_tensor(rows[:, :1], dtype=torch.float32, device=self.device)
            d['qpos'][idx] = torch.as_tensor(rows[:, 1:1 + m.nq], dtype=torch.float32, device=self.device)
            d['qvel'][idx] = torch.as_tensor(rows[:, 1 + m.nq:], dtype=torch.float32, device=self.device)
            if reset:
                for name in ('ctrl', 'qacc_warmstart', 'qfrc_applied', 'xfrc_applied'):
                    d[name][idx] = 0
                d['overflow'][idx] = 0
            mask = torch.zeros(self.num_envs, dtype=torch.int32, device=self.device)
            mask[idx] = 1
            flags = native.FLAG_NO_CONTROL | (native.FLAG_BOOTSTRAP if reset else 0) | self._route
            d.forward(mask, flags, self.stream)
            # the selected worlds' observations: cleared on reset, then sampled at once (forced)
            if reset:
                self.observer.reset(d, mask, self.stream)
            self.observer.sample(d, mask, force=True, stream=self.stream)
        self._check()

    def reset(self, id=None, *, seed=None, init_states=None):
        with self._lock:
            if self._closed:
                raise RuntimeError('environment is closed')
            self._failed = False
            if seed is not None:
                self.seed(seed)
            ids = self._ids(id)
            bank = self.initial_states if init_states is None else np.asarray(init_states)
            rows = bank[np.asarray(ids) % len(bank)] if init_states is None else bank
            self._restore(rows, ids, reset=True)
            self._evaluate(ids)
            return self._observations(ids)

    def set_init_state(self, states, id=None):
        with self._lock:
            self._open()
            ids = self._ids(id)
            self._restore(np.asarray(states), ids, reset=False)
            return self._observations(ids)

    def get_sim_state(self):
        with self._lock:
            self._open()
            self.stream.synchronize()
            d = self.data
            return np.concatenate([d['time'].double().cpu().numpy(), d['qpos'].double().cpu().numpy(),
                                   d['qvel'].double().cpu().numpy()], axis=1)

    # ------------------------------------------------------------------ stepping
    def _launch(self):
        self.observer.control_step(self.data, self.substeps, native.FLAG_POLICY_FIRST | self._route, self.stream)

    def prepare_control_graph(self):
        """Capture one control step (a single world-local launch) into a HIP graph."""
        import torch
        if self._graph is None and self._use_graph:
            g = torch.cuda.CUDAGraph()
            # warm the allocator/stream state, then capture on a side stream
            with torch.cuda.stream(self.stream):
                with torch.cuda.graph(g, stream=self.stream):
                    self._launch()
            self._graph = g
        return self

    def enqueue_action(self, actions):
        import torch
        a = np.asarray(actions, np.float64).reshape(self.num_envs, 7)
        self._actions_host.numpy()[:] = a
        with torch.cuda.stream(self.stream):
            self.data['osc_action'].copy_(self._actions_host, non_blocking=True)
            if self._use_graph:
                self.prepare_control_graph()
                self._graph.replay()
            else:
                self._launch()

    def step(self, actions):
        with self._lock:
            self._open()
            self.enqueue_action(actions)
            self._check()
            ids = list(range(self.num_envs))
            obs = self._observations(ids)
            rewards, successes = self._evaluate(ids)
            infos = [{} for _ in range(self.num_envs)]
            return obs, rewards, successes, infos

    # ------------------------------------------------------------------ predicate boundary
    def _evaluate(self, ids):
        """Rewards and successes of the selected worlds from the caller's predicates, on one
        snapshot of the fields they read (the reference evaluates its shells' _check_success on
        such a snapshot, gpu/host/backends/cuda_fp32/environment.py:200-210)."""
        if self._predicates is None:
            return np.zeros(len(ids)), np.zeros(len(ids), bool)
        rewards, successes = self._predicates(self._snapshot(self._predicate_fields), list(ids))
        return np.asarray(rewards, float).reshape(len(ids)), np.asarray(successes, bool).reshape(len(ids))

    def _snapshot(self, names=None):
        """One coherent host read of named state fields for every world, the reference's predicate
        boundary (gpu/host/backends/cuda_fp32/environment.py:215-254): body, geom and site frames and
        subtree_com shaped (nworld, n, k) (``xpos``, ``xquat``, ``xmat`` alias the body frames), the
        per-world arrays time, qpos, qvel, qacc, qacc_warmstart, ctrl, act, qfrc_applied, qfrc_bias,
        qfrc_smooth, qfrc_constraint, sensordata (nworld, n) and xfrc_applied, cfrc_ext, cfrc_int
        (nworld, nbody, 6); ``ncon`` the contact count per world and ``contact`` a list with one
        dict of ``geom1`` and ``geom2`` arrays per world.  Contacts are world-major here, so a
        masked reset leaves the other worlds' contacts in place and nothing has to be held aside.
        Raises KeyError for names it does not provide."""
        names = GOAL_FIELDS if names is None else tuple(names)
        m = self.model
        self.stream.synchronize()
        raw = self.observation_fields()
        shaped = {'body_xpos': (m.nbody, 3), 'body_xquat': (m.nbody, 4), 'body_xmat': (m.nbody, 9),
                  'geom_xpos': (m.ngeom, 3), 'geom_xmat': (m.ngeom, 9), 'site_xpos': (m.nsite, 3),
                  'site_xmat': (m.nsite, 9), 'subtree_com': (m.nbody, 3)}
        aliases = dict(xpos='body_xpos', xquat='body_xquat', xmat='body_xmat')
        roots = {'time': (), 'qpos': (m.nq,), 'qvel': (m.nv,), 'qacc': (m.nv,), 'qacc_warmstart': (m.nv,),
                 'ctrl': (m.nu,), 'act': (0,), 'qfrc_applied': (m.nv,), 'xfrc_applied': (m.nbody, 6),
                 'qfrc_bias': (m.nv,), 'qfrc_smooth': (m.nv,), 'qfrc_constraint': (m.nv,),
                 'cfrc_ext': (m.nbody, 6), 'cfrc_int': (m.nbody, 6), 'sensordata': (m.nsensordata,)}
        d = self.data
        n = self.num_envs
        result = {}
        for name in names:
            key = aliases.get(name, name)
            if key in shaped:
                result[name] = raw[key].double().cpu().numpy().reshape((n,) + shaped[key])
            elif key in roots:
                shape = roots[key]
                if key == 'act':
                    result[name] = np.zeros((n, 0))
                else:
                    size = int(np.prod(shape)) if shape else 1
                    result[name] = d[key][:, :size].double().cpu().numpy().reshape((n,) + shape)
        if 'ncon' in names or 'contact' in names:
            if m.njmax > 0:
                ncon = d['ncon'].cpu().numpy()[:, 0].astype(np.int64)
                geoms = d['contact_geom'].cpu().numpy()
            else:
                ncon, geoms = np.zeros(n, np.int64), np.zeros((n, 2), np.int32)
            if 'ncon' in names:
                result['ncon'] = ncon
            if 'contact' in names:
                result['contact'] = [dict(geom1=geoms[w, 0:2 * ncon[w]:2].copy(), geom2=geoms[w, 1:2 * ncon[w]:2].copy())
                                     for w in range(n)]
        missing = set(names) - set(result)
        if missing:
            raise KeyError('hip_mi355x boundary fields unavailable: ' + ', '.join(sorted(missing)))
        return result

    # ------------------------------------------------------------------ observations
    def observation_fields(self):
        d = self.data
        return dict(qpos=d['qpos'], qvel=d['qvel'], body_xpos=d['xpos'], body_xquat=d['xquat'],
                    body_xmat=d['xmat'], geom_xpos=d['geom_xpos'], geom_xmat=d['geom_xmat'],
                    site_xpos=d['site_xpos'], site_xmat=d['site_xmat'], subtree_com=d['subtree_com'])

    def _observations(self, ids):
        """Packed observations of the selected worlds: name -> array stacked over the worlds
        (the reference's batch_env.py:432-437), from one copy of the device's observed values."""
        self.stream.synchronize()
        values = self.observer.observed.cpu().numpy()
        packed = [self.observer.pack(values[i]) for i in ids]
        if not packed:
            return {}
        return {name: np.stack([p[name] for p in packed]) for name in packed[0]}

    # ------------------------------------------------------------------ diagnostics
    def diagnostics(self):
        self._check()
        d = self.data
        return dict(physics_backend='gpu', physics_engine=self.physics_engine, precision=self.precision,
                    actual_integration_count=d['nstep'].cpu().numpy()[:, 0].tolist(),
                    first_error=d['osc_error'].cpu().numpy()[:, 0].tolist(), substeps=self.substeps,
                    identity=dict(scene=self.model.name, **self.model.summary()),
                    capacities=dict(nconmax=self.model.nconmax, njmax=self.model.njmax),
                    upstream_status=d['overflow'].cpu().numpy()[:, 0].tolist(),
                    lds_bytes_per_world=(self.dmodel.lds_bytes_fp64() if self._route else self.dmodel.lds_bytes()))

    def work_snapshot(self):
        d = self.data
        self.stream.synchronize()
        return dict(integration_count=d['nstep'].cpu().numpy()[:, 0].tolist(),
                    first_error=d['osc_error'].cpu().numpy()[:, 0].tolist(),
                    upstream_status=d['overflow'].cpu().numpy()[:, 0].tolist())

    def close(self):
        with self._lock:
            if self._closed:
                return
            if getattr(self, 'stream', None) is not None:
                self.stream.synchronize()
            self._graph = None
            self.data = self.dmodel = self.observer = None
            self._closed = True

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __len__(self):
        return self.num_envs
