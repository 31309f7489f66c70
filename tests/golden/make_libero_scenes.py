"""Writes the LIBERO task scenes the GPU parity tests load (the reference's asset XML and BDDL files
are not on the GPU machine): each task composed by libero_hip.libero_task from the reference's
files under /root/reference, saved with libero_hip.scene_io.

    python tests/golden/make_libero_scenes.py [output folder]
"""
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1] / 'gpu-libero_amd'))

from libero_hip import libero_task, scene_io  # noqa: E402

LIBERO = Path('/root/reference/libero/libero')
TASKS = {
    # tabletop: two bowls, plate, cookies, ramekin; a wooden cabinet (3 drawers) and a flat stove
    'libero_spatial_bowl_plate': 'libero_spatial/pick_up_the_black_bowl_between_the_plate_and_the_ramekin_and_place_it_on_the_plate.bddl',
    # living room on the ground-mounted robot: groceries and a basket
    'libero_living_room_basket': 'libero_90/LIVING_ROOM_SCENE2_pick_up_the_alphabet_soup_and_put_it_in_the_basket.bddl',
    # floor scene of LIBERO-Object: seven groceries and the basket
    'libero_object_soup_basket': 'libero_object/pick_up_the_alphabet_soup_and_place_it_in_the_basket.bddl',
    # LIBERO-Goal's shared table: cabinet, wine rack, stove, bowl, plate, wine bottle, cream cheese
    'libero_goal_wine_rack': 'libero_goal/put_the_wine_bottle_on_the_rack.bddl',
    # LIBERO-10 living room: two mugs and two plates
    'libero_10_mugs_plates': 'libero_10/LIVING_ROOM_SCENE5_put_the_white_mug_on_the_left_plate_and_put_the_yellow_and_white_mug_on_the_right_plate.bddl',
}
NWORLD, SEED = 16, 0


def main(out=HERE):
    out = Path(out)
    for name, rel in TASKS.items():
        task = libero_task.compose(LIBERO / 'bddl_files' / rel, LIBERO / 'assets', nworld=NWORLD, seed=SEED)
        scene_io.save(task.scene, out / (name + '.json'))
        print(name, 'bodies', len(task.scene.bodies), 'objects', task.objects, 'fixtures', task.fixtures)


if __name__ == '__main__':
    main(*sys.argv[1:])
